"""CPU oracle for the attention path: test infrastructure, never product code.

Importable only from ``tests/``, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py``.
"""
