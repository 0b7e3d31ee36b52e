"""Per-op heuristics of the attention path (the reference's ``_opt/heuristics``)."""
