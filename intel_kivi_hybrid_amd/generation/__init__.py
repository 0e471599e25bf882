from .generate import generate
from .sampling import sample_token

__all__ = ["generate", "sample_token"]
