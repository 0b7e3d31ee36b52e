"""Shape rules and scratch buffers of the attention path (the reference's ``_opt/memory``)."""
