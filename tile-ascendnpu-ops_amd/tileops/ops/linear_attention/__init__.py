from tileops.ops.linear_attention.gdn_decode import GatedDeltaNetDecodeFwdOp
from tileops.ops.linear_attention.gdn_prefill import GatedDeltaNetPrefillFwdOp
from tileops.ops.linear_attention.gla_decode import GLADecodeOp

__all__ = ["GLADecodeOp", "GatedDeltaNetDecodeFwdOp", "GatedDeltaNetPrefillFwdOp"]
