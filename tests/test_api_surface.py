"""The Python surface a caller of the reference package finds here (CPU only).

* every ``tileops.*`` name the reference's own test files import for the
  operators built here -- tests/ops/test_{hardswish,hardsigmoid,clamp_scalar,
  clamp_min,isnan,isinf,isfinite,gelu_and_mul,gelu_tanh_and_mul,
  fused_add_layer_norm,softmax,argmax,multi_head_attention,mish,add,sub,
  bitwise_not,lerp_scalar,lerp_tensor,gla_decode}.py and
  tests/reporting/test_reporting.py -- imports from the same module path;
* Kernel metadata is truthful: every kernel is built for gfx950 only, a
  config that asks for another launch shape than the compiled one raises,
  and the rocprofv3 kernel filter each Kernel declares matches the mangled
  names of the device kernels it launches (and no other family's);
* the session-timing and msprof-compatibility helpers behave as documented.
"""

import importlib
import json
import re

import pytest
import torch

REFERENCE_TEST_IMPORTS = [
    ("tileops.benchmark.benchmark_base", "BenchmarkReport"),
    ("tileops.benchmark.msprof", "_extract_op_init_args"),
    ("tileops.benchmark.msprof", "_parse_op_basic_info"),
    ("tileops.device", "get_device_backend"),
    ("tileops.kernels.elementwise.add", "AddFwdKernel"),
    ("tileops.kernels.elementwise.bitwise_not", "BitwiseNotFwdKernel"),
    ("tileops.kernels.elementwise.clamp_scalar", "ClampScalarFwdKernel"),
    ("tileops.kernels.elementwise.gelu_and_mul", "GeluAndMulFwdKernel"),
    ("tileops.kernels.elementwise.gelu_tanh_and_mul", "GeluTanhAndMulFwdKernel"),
    ("tileops.kernels.elementwise.hardsigmoid", "HardsigmoidFwdKernel"),
    ("tileops.kernels.elementwise.hardswish", "HardswishFwdKernel"),
    ("tileops.kernels.elementwise.isfinite", "IsfiniteFwdKernel"),
    ("tileops.kernels.elementwise.isinf", "IsinfFwdKernel"),
    ("tileops.kernels.elementwise.isnan", "IsnanFwdKernel"),
    ("tileops.kernels.elementwise.lerp_scalar", "LerpScalarFwdKernel"),
    ("tileops.kernels.elementwise.mish", "MishFwdKernel"),
    ("tileops.kernels.elementwise.sub", "SubFwdKernel"),
    ("tileops.kernels.norm.fused_add_layer_norm", "FusedAddLayerNormKernel"),
    ("tileops.ops.attention.multi_head_attention", "MultiHeadAttentionFwdOp"),
    ("tileops.ops.elementwise.add", "AddFwdOp"),
    ("tileops.ops.elementwise.bitwise_not", "BitwiseNotFwdOp"),
    ("tileops.ops.elementwise.clamp_min", "ClampMinFwdOp"),
    ("tileops.ops.elementwise.clamp_scalar", "ClampScalarFwdOp"),
    ("tileops.ops.elementwise.gelu_and_mul", "GeluAndMulFwdOp"),
    ("tileops.ops.elementwise.gelu_tanh_and_mul", "GeluTanhAndMulFwdOp"),
    ("tileops.ops.elementwise.hardsigmoid", "HardsigmoidFwdOp"),
    ("tileops.ops.elementwise.hardswish", "HardswishFwdOp"),
    ("tileops.ops.elementwise.isfinite", "IsfiniteFwdOp"),
    ("tileops.ops.elementwise.isinf", "IsinfFwdOp"),
    ("tileops.ops.elementwise.isnan", "IsnanFwdOp"),
    ("tileops.ops.elementwise.lerp_scalar", "LerpFwdOp"),
    ("tileops.ops.elementwise.lerp_tensor", "LerpTensorFwdOp"),
    ("tileops.ops.elementwise.mish", "MishFwdOp"),
    ("tileops.ops.elementwise.sub", "SubFwdOp"),
    ("tileops.ops.linear_attention.gla_decode", "GLADecodeOp"),
    ("tileops.ops.norm.fused_add_layer_norm", "FusedAddLayerNormFwdOp"),
    ("tileops.ops.reduction.argmax", "ArgmaxFwdOp"),
    ("tileops.ops.reduction.softmax", "LogSumExpFwdOp"),
    ("tileops.reporting.analyzer", "analyze_run"),
    ("tileops.reporting.cli", "_parser"),
    ("tileops.reporting.collector", "parse_junit_report"),
    ("tileops.reporting.report", "write_reports"),
    ("tileops.reporting.runner", "resolve_operator"),
    ("tileops.reporting.runner", "run_operator"),
    ("tileops.reporting.session_timing", "attach_session_timing"),
    ("tileops.reporting.session_timing", "parse_session_timing"),
    ("tileops.testing", "record_check_result"),
    ("tileops.testing.test_base", "TestBase"),
    ("tileops.testing.test_base", "allclose_compare"),
    ("tileops.workloads.attention", "MhaFwdWorkload"),
    ("tileops.workloads.elementwise", "BitwiseNotWorkload"),
    ("tileops.workloads.elementwise", "IsfiniteWorkload"),
    ("tileops.workloads.elementwise", "IsinfWorkload"),
    ("tileops.workloads.elementwise", "IsnanWorkload"),
    ("tileops.workloads.linear_attention", "GLADecodeWorkload"),
    ("tileops.workloads.linear_attention", "gla_decode_tolerance"),
    ("tileops.workloads.norm", "FusedAddLayerNormWorkload"),
    ("tileops.workloads.reduction", "ArgmaxWorkload"),
    ("tileops.workloads.reduction", "LogSumExpWorkload"),
    ("tileops.workloads.workload_base", "FixtureBase"),
    ("tileops.workloads.workload_base", "RandnWorkload"),
]


@pytest.mark.parametrize("module, name", REFERENCE_TEST_IMPORTS)
def test_reference_test_imports_resolve(module, name):
    assert hasattr(importlib.import_module(module), name), f"{module}.{name}"


# Representative mangled names of the device kernels in libtileops_hip.so, by the
# Kernel classes that launch them.
# rocprofv3 records the demangled name where its demangler succeeds and the
# mangled one where it fails (_Float16 / __bf16 template arguments): both forms
_MANGLED = {
    "unary": ["_ZN7tileops16unary_vec_kernelIDF16_Li0EEEvPKT_PS1_lffi",
              "_ZN7tileops19unary_scalar_kernelIfLi2EEEvPKT_PS1_llffi",
              "void tileops::unary_scalar_kernel<float, 2>(float const*, float*, long, long)"],
    "isfp": ["_ZN7tileops15isfp_vec_kernelIfLi0EEEvPKT_Phl",
             "_ZN7tileops18isfp_scalar_kernelIfLi1EEEvPKT_Phll"],
    "gated": ["_ZN7tileops21gated_gelu_vec_kernelIDF16b_Li0ELi2EEEvPKT_PS1_ll",
              "_ZN7tileops24gated_gelu_scalar_kernelIfLi1EEEvPKT_PS1_ll",
              "void tileops::gated_gelu_vec_kernel<float, 0>(float const*, float*, unsigned int, unsigned int)",
              "_ZN7tileops22gated_gelu_rows_kernelIDF16b_Li1ELi2EEEvPKT_PS1_ll"],
    "bcast": ["_ZN7tileops16bcast_vec_kernelIfLi0EEEvPKT_S3_S3_PS1_lf",
              "_ZN7tileops18bcast_inner_kernelIDF16_Li1EjEEvPKT_S3_S3_PS1_T1_S5_f",
              "_ZN7tileops16bcast_any_kernelIfLi2EEEvPKT_S3_S3_PS1_llfNS_9BcastDescE"],
    "bitnot": ["_ZN7tileops17bitnot_vec_kernelEPKDv4_jPS0_lj",
               "_ZN7tileops18bitnot_byte_kernelEPKhPhllj"],
    "ln": ["_ZN7tileops24fused_add_ln_wave_kernelIDF16b_Li2ELi16ELi4EEEvPKT_S3_PKvS5_PS1_S6_lf",
           "_ZN7tileops25fused_add_ln_block_kernelIffLi5EEEvPKT_S3_PKT0_S6_PS1_S7_ifb",
           "tileops::fused_add_ln_block_kernel<float, float, 5>(float const*)",
           "_ZN7tileops27fused_add_ln_generic_kernelIfLi0EEEvPKT_S3_PKvS5_PS1_S6_llf"],
    "row": ["_ZN7tileops17row_reduce_kernelIfLi0ELi1ELi4ELb1EEEvPKT_Pvll",
            "void tileops::row_reduce_kernel<float, 0, 1, 4, true>(float const*, void*, long, long)"],
    "mha": ["_ZN7tileops3mha14mha_fwd_kernelIDF16b_Li128ELb1ELi64ELb0EEEvPKT_S4_S4_PS2_Pfiiiiififf"],
    "gdn": ["_ZN7tileops3gdn16gdn_fused_kernelILi4EEEvNS0_4ArgsE",
            "_ZN7tileops3gdn16gdn_fused_kernelILi8EEEvNS0_4ArgsE",
            "void tileops::gdn::gdn_fused_kernel<8>(tileops::gdn::Args)",
            "_ZN7tileops3gdn21gdn_copy_state_kernelEPKfPfl",
            "_ZN7tileops3gdn18gdn_compose_kernelILi2EEEvNS0_4ArgsE"],
    "gla": ["_ZN7tileops3gla17gla_decode_kernelIDF16bLb1EEEvPKT_S4_S4_S4_PKfPS2_Pfiiif",
            "_ZN7tileops3gla22gla_decode_rows_kernelIDF16bLi16ELi8ELb0EEEvPKT_S4_S4_S4_S4_PS2_S5_if"],
    "gdnd": ["_ZN7tileops4gdnd17gdn_decode_kernelIDF16bLi16ELi8ELb1EEEvPKT_S4_S4_PKfS6_S6_PS2_Pfif",
             "void tileops::gdnd::gdn_decode_kernel<float, 8, 8>(float const*)"],
}


def _kernel_groups():
    from tileops.kernels.attention.multi_head_attention import GQAPrefillFwdKernel
    from tileops.kernels.elementwise.add import AddFwdKernel
    from tileops.kernels.elementwise.bitwise_not import BitwiseNotFwdKernel
    from tileops.kernels.elementwise.gelu_and_mul import GeluAndMulFwdKernel
    from tileops.kernels.elementwise.hardswish import HardswishFwdKernel
    from tileops.kernels.elementwise.isnan import IsnanFwdKernel
    from tileops.kernels.elementwise.lerp_scalar import LerpScalarFwdKernel
    from tileops.kernels.elementwise.lerp_tensor import LerpTensorFwdKernel
    from tileops.kernels.elementwise.sub import SubFwdKernel
    from tileops.kernels.linear_attention.gdn_decode import GDNDecodeKernel
    from tileops.kernels.linear_attention.gdn_prefill import GDNPrefillFwdKernel
    from tileops.kernels.linear_attention.gla_decode import GLADecodeKernel
    from tileops.kernels.norm.fused_add_layer_norm import FusedAddLayerNormKernel
    from tileops.kernels.reduction.argmax import ArgreduceKernel
    from tileops.kernels.reduction.logsumexp import LogSumExpKernel

    return [(HardswishFwdKernel, "unary"), (IsnanFwdKernel, "isfp"),
            (GeluAndMulFwdKernel, "gated"), (AddFwdKernel, "bcast"), (SubFwdKernel, "bcast"),
            (LerpScalarFwdKernel, "bcast"), (LerpTensorFwdKernel, "bcast"),
            (BitwiseNotFwdKernel, "bitnot"), (FusedAddLayerNormKernel, "ln"),
            (LogSumExpKernel, "row"), (ArgreduceKernel, "row"), (GQAPrefillFwdKernel, "mha"),
            (GDNPrefillFwdKernel, "gdn"), (GLADecodeKernel, "gla"), (GDNDecodeKernel, "gdnd")]


@pytest.mark.parametrize("idx", range(15))
def test_profile_regex_matches_own_kernels_only(idx):
    cls, group = _kernel_groups()[idx]
    assert cls.supported_archs == ["gfx950"], cls.__name__
    pat = re.compile(cls.profile_kernel_name)
    for g, names in _MANGLED.items():
        for n in names:
            assert bool(pat.search(n)) == (g == group), (cls.__name__, n)


def test_rocprof_filter_resolves_through_ops():
    from tileops.benchmark.rocprof import _resolve_kernel_regex
    from tileops.ops.elementwise.lerp_tensor import LerpTensorFwdOp
    from tileops.ops.reduction.argmax import ArgmaxFwdOp

    op = LerpTensorFwdOp(input=(4,), end=(4,), weight=(4,), dtype=torch.float32)
    assert _resolve_kernel_regex(op, None)[0] == op.kernel.profile_kernel_name
    # an Op whose kernel is built lazily resolves through its kernel map
    am = ArgmaxFwdOp(dtype=torch.float32, dim=-1)
    assert re.search(_resolve_kernel_regex(am, None)[0], _MANGLED["row"][0])
    assert _resolve_kernel_regex(op, "explicit")[0] == "explicit"


def test_config_overrides_must_match_the_compiled_kernel(capsys):
    from tileops.kernels.attention.multi_head_attention import GQAPrefillFwdKernel
    from tileops.kernels.elementwise.hardswish import HardswishFwdKernel

    k = HardswishFwdKernel(64, torch.float16, config={"threads": 256, "vector_bytes": None})
    assert k.config == k.default_config
    with pytest.raises(ValueError, match="compiled kernel uses"):
        HardswishFwdKernel(64, torch.float16, config={"packs_per_thread": 4})
    with pytest.raises(ValueError, match="unknown config keys"):
        HardswishFwdKernel(64, torch.float16, config={"unroll": 4})
    mha = GQAPrefillFwdKernel(1, 2, 2, 256, 256, 128, True, torch.bfloat16)
    assert mha.config["block_m"] == 256 and mha.config["block_n"] == 128
    assert mha.config["num_stages"] == 2
    mha64 = GQAPrefillFwdKernel(1, 2, 2, 256, 256, 64, True, torch.bfloat16)
    assert mha64.config["block_n"] == 64 and mha64.config["num_stages"] == 3
    with pytest.raises(ValueError, match="block_m=128"):
        GQAPrefillFwdKernel(1, 2, 2, 256, 256, 128, True, torch.bfloat16, config={"block_m": 128})


def test_msprof_csv_parser(tmp_path):
    from tileops.benchmark.msprof import _parse_op_basic_info

    for op, idx, dur in (("Main", 0, "8.5"), ("Aux", 0, "2.0"), ("Main", 1, "bad")):
        d = tmp_path / "OPPROF_x" / op / str(idx)
        d.mkdir(parents=True)
        (d / f"OpBasicInfo_{idx}.csv").write_text(f"Op Name,Task Duration(us)\n{op},{dur}\n")
    durations, first, names = _parse_op_basic_info(tmp_path)
    # sorted path order: Aux/0, Main/0, Main/1 (non-numeric skipped)
    assert durations == [2.0, 8.5] and first == "Aux" and names == ["Aux", "Main"]
    with pytest.raises(FileNotFoundError):
        _parse_op_basic_info(tmp_path / "none")


def _timing_file(path, operator, total=3661.25):
    path.parent.mkdir(parents=True, exist_ok=True)
    doc = {"schema_version": 1, "operator": operator, "total_duration_s": total,
           "breakdown": [{"name": "Integration", "duration_s": 61.25, "ratio_percent": 1.67,
                          "detail": "log"}]}
    path.write_text("<!-- TILEOPS_SESSION_TIMING_V1\n" + json.dumps(doc) + "\n-->\n# Timing\n")


def test_session_timing_parse_attach_render(tmp_path):
    from tileops.reporting.cli import _parser
    from tileops.reporting.report import render_html, render_markdown
    from tileops.reporting.session_timing import (
        attach_session_timing, format_duration, parse_session_timing)

    src = tmp_path / "SESSION_TIMING_ANALYSIS.md"
    _timing_file(src, "DemoOp")
    ok = parse_session_timing(src, "DemoOp")
    assert ok["status"] == "available" and ok["total_duration_s"] == 3661.25
    assert ok["breakdown"][0]["name"] == "Integration"
    bad = parse_session_timing(src, "OtherOp")
    assert bad["status"] == "invalid" and "operator mismatch" in bad["reason"]
    _timing_file(src, "DemoOp", total=-1)
    assert parse_session_timing(src, "DemoOp")["status"] == "invalid"
    assert parse_session_timing(tmp_path / "nope.md", "DemoOp")["status"] == "missing"
    assert format_duration(3661.25) == "1h01m01s" and format_duration(None) == "N/A"

    root = tmp_path / "pkg"
    meta = root / "tileops" / "kernels" / "demo" / "alpha" / ".migration_meta.json"
    meta.parent.mkdir(parents=True)
    meta.write_text(json.dumps({"op_name": "AlphaOp", "op_slug": "alpha_task"}))
    _timing_file(tmp_path / "alpha_task" / "SESSION_TIMING_ANALYSIS.md", "AlphaOp")
    run = {"operator": "all", "status": "passed", "summary": {}, "warnings": [],
           "operators": [{"operator": "AlphaOp"}, {"operator": "BetaOp"}],
           "performance": {"cases": []}, "correctness": {"cases": []},
           "benchmark_tests": {"cases": []}}
    plain_md = render_markdown(dict(run))
    attach_session_timing(run, root=root, operator_catalog=[], enabled=False)
    assert "session_timing" not in run and "Session Timing" not in plain_md
    attach_session_timing(run, root=root, operator_catalog=[], enabled=True)
    recs = run["session_timing"]["operators"]
    assert recs["AlphaOp"]["status"] == "available" and recs["BetaOp"]["status"] == "missing"
    md, page = render_markdown(run), render_html(run)
    assert "| Operator | Total Time |" in md and "1h01m01s" in md
    assert "Timing data unavailable: SESSION_TIMING_ANALYSIS.md not found" in md
    assert "Session Timing / Session 耗时" in page and "Total Time / 总时间" in page

    args = _parser().parse_args(["run", "--all", "--with-session-timing"])
    assert args.with_session_timing is True
    assert _parser().parse_args(["render", "r.json", "--with-session-timing"]).with_session_timing
