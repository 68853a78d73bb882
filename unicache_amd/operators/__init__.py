"""Physical-cache operators of the UniCache engine on MI355X."""

from .builtin import KIVIQuantizationOperator, asymmetric_fake_quant, kivi_fake_quant_key, kivi_fake_quant_value
from .physical import (
    H2OPhysicalGQAOperator,
    KIVIPackedQuantizationOperator,
    per_kv_head_scores_from_probs,
    per_kv_head_scores_from_qk,
)

__all__ = [
    "H2OPhysicalGQAOperator",
    "KIVIPackedQuantizationOperator",
    "KIVIQuantizationOperator",
    "asymmetric_fake_quant",
    "kivi_fake_quant_key",
    "kivi_fake_quant_value",
    "per_kv_head_scores_from_probs",
    "per_kv_head_scores_from_qk",
]
