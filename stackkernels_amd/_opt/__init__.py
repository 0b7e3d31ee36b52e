"""Device profile and kernel-configuration introspection for the attention path.

The reference's ``stackkernels._opt`` (``src/stackkernels/_opt/``) picks Triton
launch configurations from a ``DeviceProfile``.  Here the configurations are the
gfx950 table compiled into ``libsk_attn.so``; ``pick`` reports them (and the
grid, occupancy and scratch they imply) through the library's
``sk_kernel_config``, so the answer is the configuration that actually runs.
"""
