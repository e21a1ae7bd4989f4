"""Manifest loader, workload contract and roofline formulas.

The loader contract follows examples/TileOPs/tileops/manifest/__init__.py:28-89;
the roofline figures of the MI355X headline rows are pinned to the closed
forms of the byte / flop counts (hand-evaluated constants), and every Op's
``eval_roofline`` is checked against its manifest formula on every workload
whose shape the Op binds at construction.
"""

import pytest
import torch

from tileops.benchmark.benchmark_base import workloads_to_params
from tileops.manifest import (
    WORKLOAD_RESERVED_KEYS,
    load_manifest,
    load_workloads,
    manifest_files,
    single_input_workload_contract,
)
from tileops.manifest.roofline import manifest_roofline, reduced_dims

HOT_PATH_OPS = {
    "HardswishFwdOp", "HardsigmoidFwdOp", "ClampScalarFwdOp", "IsnanFwdOp", "IsinfFwdOp",
    "IsfiniteFwdOp", "GeluAndMulFwdOp", "GeluTanhAndMulFwdOp", "FusedAddLayerNormFwdOp",
    "LogSumExpFwdOp", "ArgmaxFwdOp", "MultiHeadAttentionFwdOp", "GatedDeltaNetPrefillFwdOp",
}
# ops beyond the hot path built on its kernels (the clamp kernel without an upper bound)
WIDENED_OPS = {"AddFwdOp", "BitwiseNotFwdOp", "ClampMinFwdOp", "GLADecodeOp", "LerpFwdOp",
               "LerpTensorFwdOp", "MishFwdOp", "SubFwdOp", "GatedDeltaNetDecodeFwdOp"}


def test_manifest_holds_the_hot_path_ops():
    assert set(load_manifest()) == HOT_PATH_OPS | WIDENED_OPS
    assert [p.name for p in manifest_files()] == sorted(p.name for p in manifest_files())


def test_every_entry_declares_sources_that_exist():
    import os

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for name, entry in load_manifest().items():
        src = entry["source"]
        for key in ("kernel", "op", "test", "bench"):
            assert os.path.exists(os.path.join(root, src[key])), (name, key, src[key])
        assert entry["workloads"], name
        for w in entry["workloads"]:
            assert w["dtypes"] and w["label"], (name, w)


def test_load_workloads_unknown_op():
    with pytest.raises(KeyError, match="not found in ops manifest"):
        load_workloads("NoSuchFwdOp")


def test_duplicate_op_is_rejected(tmp_path, monkeypatch):
    import tileops.manifest as mf

    (tmp_path / "a.yaml").write_text("FooOp: {workloads: []}\n")
    (tmp_path / "b.yaml").write_text("FooOp: {workloads: []}\n")
    monkeypatch.setattr(mf, "_DIR", tmp_path)
    mf.load_manifest.cache_clear()
    try:
        with pytest.raises(ValueError, match="duplicate op 'FooOp' in b.yaml"):
            mf.load_manifest()
    finally:
        monkeypatch.undo()
        mf.load_manifest.cache_clear()


def test_top_level_must_be_mapping(tmp_path, monkeypatch):
    import tileops.manifest as mf

    (tmp_path / "a.yaml").write_text("- 1\n- 2\n")
    monkeypatch.setattr(mf, "_DIR", tmp_path)
    mf.load_manifest.cache_clear()
    try:
        with pytest.raises(ValueError, match="top-level mapping"):
            mf.load_manifest()
    finally:
        monkeypatch.undo()
        mf.load_manifest.cache_clear()


def test_single_input_contract():
    sig = load_manifest()["ClampScalarFwdOp"]["signature"]
    key, allowed = single_input_workload_contract(sig)
    assert key == "input_shape"
    assert allowed == {"min", "max", "input_shape"} | WORKLOAD_RESERVED_KEYS
    assert single_input_workload_contract(load_manifest()["MultiHeadAttentionFwdOp"]["signature"]) is None


def test_workloads_to_params_ids_and_extras():
    params = workloads_to_params("ClampScalarFwdOp", include_extra=True)
    ids = [p.id for p in params]
    assert ids[:3] == ["smoke-1m-float32", "smoke-1m-float16", "smoke-1m-bfloat16"]
    shape, dtype, extra = params[0].values
    assert shape == (1048576,) and dtype is torch.float32 and extra == {"min": -0.5, "max": 0.5}
    assert "16M-max-only-float16" in ids
    with pytest.raises(KeyError, match="multi-input"):
        workloads_to_params("MultiHeadAttentionFwdOp")


def test_reduced_dims():
    assert reduced_dims((4, 128, 4096), [0, 2]) == [0, 2]
    assert reduced_dims((4, 128, 4096), -1) == [2]
    assert reduced_dims((4, 5), None) == [0, 1]
    assert reduced_dims((4, 5), [-1, 1]) == [1]


# (op, label, dtype) -> (flops, bytes): closed forms evaluated by hand, e.g.
# hardswish fp16 8192^2: bytes 2*N*2 = 268,435,456; GDN: (6C^2K + 4C^2V +
# 6CKV + C^3//3) * (8192/64)*4*16 = 95,205,105,664.
PINNED = [
    ("HardswishFwdOp", "mi355x-headline", "float16", 4 * 8192 * 8192, 268_435_456),
    ("HardsigmoidFwdOp", "mi355x-headline", "float16", 3 * 8192 * 8192, 268_435_456),
    ("ClampScalarFwdOp", "mi355x-headline", "float16", 8192 * 8192, 268_435_456),
    ("IsnanFwdOp", "mi355x-headline", "float32", 8192 * 8192, 335_544_320),
    ("GeluAndMulFwdOp", "mi355x-headline", "bfloat16", 6 * 16384 * 11008, 1_082_130_432),
    ("GeluTanhAndMulFwdOp", "mi355x-headline", "bfloat16", 10 * 16384 * 11008, 1_082_130_432),
    ("FusedAddLayerNormFwdOp", "mi355x-headline", "bfloat16", 8 * 32768 * 4096, 1_073_774_592),
    ("FusedAddLayerNormFwdOp", "llama-8b-prefill", "bfloat16", 8 * 2048 * 4096, 67_125_248),
    ("LogSumExpFwdOp", "mi355x-headline", "float32", 4 * 32768 * 4096, 537_001_984),
    ("LogSumExpFwdOp", "3d-multidim-reduce", "float16", 4 * 128 * 16384, (128 * 16384 + 128) * 2),
    ("ArgmaxFwdOp", "mi355x-headline", "float32", 32768 * 4096, 537_133_056),
    ("ArgmaxFwdOp", "3d-non-last-axis-argmax", "float16", 4 * 128 * 4096, 4 * 128 * 4096 * 2 + 128 * 4096 * 8),
    ("MultiHeadAttentionFwdOp", "mi355x-headline", "bfloat16", 2_199_023_255_552, 1_073_741_824),
    ("MultiHeadAttentionFwdOp", "mi355x-headline-causal", "bfloat16", 1_099_511_627_776, 1_073_741_824),
    ("GatedDeltaNetPrefillFwdOp", "mi355x-headline", "bfloat16", 95_205_105_664, 545_259_520),
    ("GatedDeltaNetDecodeFwdOp", "mi355x-headline", "bfloat16", 948_961_280, 1_082_195_968),
]


@pytest.mark.parametrize("op, label, dtype, flops, nbytes", PINNED)
def test_manifest_roofline_pinned(op, label, dtype, flops, nbytes):
    (w,) = [w for w in load_workloads(op) if w["label"] == label]
    assert manifest_roofline(op, w, dtype) == (flops, nbytes)


def _static_ops():
    from tileops.ops.attention.multi_head_attention import MultiHeadAttentionFwdOp
    from tileops.ops.elementwise.add import AddFwdOp
    from tileops.ops.elementwise.bitwise_not import BitwiseNotFwdOp
    from tileops.ops.elementwise.clamp_min import ClampMinFwdOp
    from tileops.ops.elementwise.clamp_scalar import ClampScalarFwdOp
    from tileops.ops.elementwise.gelu_and_mul import GeluAndMulFwdOp
    from tileops.ops.elementwise.gelu_tanh_and_mul import GeluTanhAndMulFwdOp
    from tileops.ops.elementwise.hardsigmoid import HardsigmoidFwdOp
    from tileops.ops.elementwise.hardswish import HardswishFwdOp
    from tileops.ops.elementwise.isfinite import IsfiniteFwdOp
    from tileops.ops.elementwise.isinf import IsinfFwdOp
    from tileops.ops.elementwise.isnan import IsnanFwdOp
    from tileops.ops.elementwise.lerp_scalar import LerpFwdOp
    from tileops.ops.elementwise.lerp_tensor import LerpTensorFwdOp
    from tileops.ops.elementwise.mish import MishFwdOp
    from tileops.ops.elementwise.sub import SubFwdOp
    from tileops.ops.linear_attention.gdn_decode import GatedDeltaNetDecodeFwdOp
    from tileops.ops.linear_attention.gdn_prefill import GatedDeltaNetPrefillFwdOp
    from tileops.ops.linear_attention.gla_decode import GLADecodeOp

    def flat(cls):
        def make(w, dt):
            n = 1
            for s in w["input_shape"]:
                n *= s
            kw = {k: w[k] for k in ("min", "max") if k in w}
            return cls(N_total=n, dtype=dt, **kw)
        return make

    def gated(cls):
        return lambda w, dt: cls(M=w["M"], N=w["N"], dtype=dt)

    return {
        "HardswishFwdOp": flat(HardswishFwdOp),
        "HardsigmoidFwdOp": flat(HardsigmoidFwdOp),
        "ClampScalarFwdOp": flat(ClampScalarFwdOp),
        "ClampMinFwdOp": flat(ClampMinFwdOp),
        "BitwiseNotFwdOp": flat(BitwiseNotFwdOp),
        "IsnanFwdOp": flat(IsnanFwdOp),
        "MishFwdOp": flat(MishFwdOp),
        "IsinfFwdOp": flat(IsinfFwdOp),
        "IsfiniteFwdOp": flat(IsfiniteFwdOp),
        "GeluAndMulFwdOp": gated(GeluAndMulFwdOp),
        "GeluTanhAndMulFwdOp": gated(GeluTanhAndMulFwdOp),
        "MultiHeadAttentionFwdOp": lambda w, dt: MultiHeadAttentionFwdOp(
            w["q_shape"][0], w["q_shape"][2], w["q_shape"][1], w["q_shape"][3],
            w.get("is_causal", True), dt),
        "GLADecodeOp": lambda w, dt: GLADecodeOp(w["B"], w["H"], w["DK"], w["DV"],
                                                 scale=w.get("scale", -1.0), dtype=dt),
        "AddFwdOp": lambda w, dt: AddFwdOp(input=tuple(w["input_shape"]),
                                           other=tuple(w["other_shape"]), dtype=dt),
        "SubFwdOp": lambda w, dt: SubFwdOp(input=tuple(w["input_shape"]),
                                           other=tuple(w["other_shape"]), dtype=dt),
        "LerpFwdOp": lambda w, dt: LerpFwdOp(input=tuple(w["input_shape"]),
                                             end=tuple(w["end_shape"]), dtype=dt),
        "LerpTensorFwdOp": lambda w, dt: LerpTensorFwdOp(
            input=tuple(w["input_shape"]), end=tuple(w["input_shape"]),
            weight=tuple(w["input_shape"]), dtype=dt),
        "GatedDeltaNetPrefillFwdOp": lambda w, dt: GatedDeltaNetPrefillFwdOp(
            w["batch"], w["seq_len"], w["heads"], w["dim_k"], w["dim_v"], dtype=dt),
        "GatedDeltaNetDecodeFwdOp": lambda w, dt: GatedDeltaNetDecodeFwdOp(
            w["batch"], w["heads"], w["dim_k"], w["dim_v"], dtype=dt),
    }


def test_op_eval_roofline_matches_manifest_formula():
    makers = _static_ops()
    checked = 0
    for op_name, make in makers.items():
        for w in load_workloads(op_name):
            for d in w["dtypes"]:
                dt = getattr(torch, d)
                assert make(w, dt).eval_roofline() == manifest_roofline(op_name, w, dt), (op_name, w, d)
                checked += 1
    assert checked > 80
