"""Flash attention and the teaching attention (examples/flash_attention in the reference)."""

from .attention import attention_target, causal_policy
from .simple import simple_attention

__all__ = ["attention_target", "causal_policy", "simple_attention"]
