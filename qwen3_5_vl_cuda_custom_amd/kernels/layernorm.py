from .norms import layernorm  # noqa: F401
