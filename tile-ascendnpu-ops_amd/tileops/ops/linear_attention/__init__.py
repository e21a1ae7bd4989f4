from tileops.ops.linear_attention.gdn_prefill import GatedDeltaNetPrefillFwdOp

__all__ = ["GatedDeltaNetPrefillFwdOp"]
