"""MI355X-native Co-ALiBi attention (drop-in for Nathancgy/Co-ALIBI's co_alibi_attn)."""
from .co_alibi_attn import co_alibi_attention, co_alibi_decode

__all__ = ["co_alibi_attention", "co_alibi_decode"]
