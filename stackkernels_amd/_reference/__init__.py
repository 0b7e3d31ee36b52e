"""PyTorch reference implementations (the CPU / ``reference``-backend path)."""
