"""KV-cache kernels (launchers over ``libsk_attn.so``)."""
