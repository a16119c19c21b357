from .elementwise import swiglu  # noqa: F401
