from .elementwise import gelu_tanh  # noqa: F401
