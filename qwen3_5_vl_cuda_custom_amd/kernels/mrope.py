from .rotary import apply_mrope  # noqa: F401
