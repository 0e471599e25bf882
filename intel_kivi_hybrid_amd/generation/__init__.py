from .generate import generate, generate_packed
from .sampling import sample_token

__all__ = ["generate", "generate_packed", "sample_token"]
