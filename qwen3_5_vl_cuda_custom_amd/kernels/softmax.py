from .norms import softmax  # noqa: F401
