"""bench.py's contract pieces that need no GPU: the multi-GPU refusal, and
the counter-measured HBM bytes it attaches to its roofline and kernel rows,
read from the committed traffic profile."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# every kernel an encoder layer launches (the roofline candidates), the
# bandwidth-bound kernels held to the HBM target, and their same-byte copies
PROFILED = ("qkv_attn_ln_s128", "out_proj_res_stats", "ffn_up_ln", "ffn_down_res_stats",
            "ffn_up_ln_frag", "ffn_down_res_stats_frag", "qkv_attn_ln_s128_frag",
            "out_proj_res_stats_frag", "int8_ffn_up_frag", "int8_ffn_down_res_stats_frag",
            "int8_ffn_down_res_stats", "add_layernorm_q8_res_ln", "attn_s512",
            "add_layernorm", "add_layernorm_s512", "bias_gelu", "bias_gelu_s512",
            "copy_18.9MB", "copy_50.3MB", "copy_75.5MB", "copy_201MB")


@pytest.mark.parametrize("name", PROFILED)
def test_profiled_traffic_present(name):
    import bench

    assert name in bench.STEP_KERNELS or name in _case_names()
    t = bench.pmc_traffic(name)
    assert t is not None and t > 0, name


def test_bandwidth_kernels_move_their_algorithmic_bytes():
    """The LN/GELU rows of the profile: counter traffic equals the bytes the
    kernel must move (inputs read once, output written once) within 1%."""
    import bench

    M, H, F = 4096, 768, 3072
    alg = {
        "add_layernorm": 3 * M * H * 2,
        "add_layernorm_s512": 3 * 4 * M * H * 2,
        "bias_gelu": 2 * M * F * 2,
        "bias_gelu_s512": 2 * 4 * M * F * 2,
    }
    for name, nbytes in alg.items():
        assert abs(bench.pmc_traffic(name) / nbytes - 1.0) < 0.01, name


def test_unknown_case_has_no_traffic():
    import bench

    assert bench.pmc_traffic("no_such_kernel") is None


def test_multi_gpu_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       cwd=ROOT, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr


def _case_names():
    """Case names of bench.kernel_cases, read from its source (building the
    cases needs a GPU)."""
    import re

    src = open(os.path.join(ROOT, "bench.py")).read()
    body = src[src.index("def kernel_cases("):src.index("\ndef ", src.index("def kernel_cases(") + 1)]
    table = body[body.rindex("return {"):]
    return set(re.findall(r'^\s+"([A-Za-z0-9_.]+)": [a-z_0-9]+\(', table, re.M))
