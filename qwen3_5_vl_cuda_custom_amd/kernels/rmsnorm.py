from .norms import rmsnorm  # noqa: F401
