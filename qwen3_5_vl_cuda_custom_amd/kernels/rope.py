from .rotary import apply_rope  # noqa: F401
