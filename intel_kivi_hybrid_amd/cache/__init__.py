from .manager import KiviCache
from .packed_cache import KIVI_ATTENTION, KiviPackedCache, packed_attention, register_packed_attention

__all__ = ["KIVI_ATTENTION", "KiviCache", "KiviPackedCache", "packed_attention",
           "register_packed_attention"]
