from .manager import KiviCache

__all__ = ["KiviCache"]
