from .bagel import merge_attention_summaries, run_batched_physical_attention, run_fused_mixed_attention

__all__ = ["merge_attention_summaries", "run_batched_physical_attention", "run_fused_mixed_attention"]
