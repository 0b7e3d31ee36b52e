"""Kernel launchers (ctypes over libsk_attn.so)."""
