from .bagel import merge_attention_summaries

__all__ = ["merge_attention_summaries"]
