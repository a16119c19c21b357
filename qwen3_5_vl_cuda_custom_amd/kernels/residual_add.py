from .elementwise import residual_add  # noqa: F401
