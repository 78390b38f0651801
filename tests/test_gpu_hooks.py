"""GPU: the graph hooks route a PyTorch BERT layer through the HIP kernels.
FX rewriting and torch.compile(backend=zenith) must produce a graph whose
compute calls are all HIP leaves, and its output must match the oracle's
fp32 layer at the encoder bar (norm-relative and elementwise 2e-2). The
registry + dispatcher path is checked on the fused op types against the
oracle at the fp16 bar."""

import numpy as np
import pytest
import torch

from oracle import bert as obert
from oracle import ops
from tests.conftest import fp16_tol
from zenith_amd import synthetic

pytestmark = pytest.mark.gpu


def _r16(w):
    return {k: synthetic.round_f16(v) for k, v in w.items()}


def _check(y, ref, bar=2e-2):
    rel = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
    worst = float(np.max(np.abs(y - ref) - (bar + bar * np.abs(ref))))
    assert rel <= bar and worst <= 0, (rel, worst)


def _layer(dev, B=2, S=128):
    from zenith_amd.torch_bert import TorchBertLayer

    w = _r16(synthetic.bert_weights(1, seed=11)[0])
    x = synthetic.round_f16(synthetic.hidden_states(B, S, seed=11))
    m = TorchBertLayer(w).to(dev).half().eval()
    return m, w, x, torch.from_numpy(x).to(dev, torch.float16)


def test_fx_rewritten_bert_layer(dev):
    from zenith_amd.hooks import fx_optimizer as O

    m, w, x, xt = _layer(dev)
    gm = torch.fx.symbolic_trace(m)
    opt = O.FXOptimizer(strict=True)
    gm = opt.optimize(gm, [xt])
    t = O.replaced_targets(gm)
    assert t.count("hip_linear") == 5 and t.count("hip_linear_gelu") == 1
    assert t.count("hip_add_layernorm_eps") == 2 and t.count("hip_flash_attention") == 1
    with torch.no_grad():
        y = gm(xt).float().cpu().numpy()
    _check(y, obert.bert_layer(x, w))


def test_torch_compile_backend(dev):
    import torch._dynamo

    from zenith_amd.hooks import backend, fx_optimizer as O

    m, w, x, xt = _layer(dev)
    torch._dynamo.reset()
    be = backend.create_compile_backend(precision="fp16")
    cm = torch.compile(m, backend=be, dynamic=False)
    with torch.no_grad():
        y = cm(xt).float().cpu().numpy()
    st = be.last_stats
    assert st is not None and st.patterns_replaced >= 9, st
    _check(y, obert.bert_layer(x, w))


def test_torch_compile_backend_padding_mask(dev):
    """A padded batch: the boolean [B, 1, S, S] mask HF BERT's SDPA path
    builds reaches the masked HIP attention kernel through torch.compile
    (no SDPA left in the graph), and the layer matches the oracle layer with
    the same key-padding lengths."""
    import torch._dynamo

    from zenith_amd.hooks import backend
    from zenith_amd.torch_bert import MaskedTorchBertLayer

    _, w, x, xt = _layer(dev)
    m = MaskedTorchBertLayer(w).to(dev).half().eval()
    B, S = x.shape[:2]
    lens = np.array([S, S // 2 + 5], np.int32)
    keep = torch.arange(S, device=dev)[None, :] < torch.from_numpy(lens).to(dev)[:, None]
    mask = keep[:, None, None, :].expand(B, 1, S, S)
    torch._dynamo.reset()
    be = backend.create_compile_backend(precision="fp16")
    cm = torch.compile(m, backend=be, dynamic=False)
    with torch.no_grad():
        y = cm(xt, mask).float().cpu().numpy()
    st = be.last_stats
    assert st is not None and "structural_sdpa_to_flash" in st.passes_applied, st
    _check(y, obert.bert_layer(x, w, lens))


def test_dispatcher_fused_ops(dev):
    from zenith_amd.hooks import ExecutionContext, KernelDispatcher, Node, Precision

    w = _r16(synthetic.bert_weights(1, seed=12)[0])
    M, H = 256, 768
    x = synthetic.round_f16(synthetic.normal((M, H), tag=40))
    r = synthetic.round_f16(synthetic.normal((M, H), tag=41))
    T = {k: torch.from_numpy(v).to(dev, torch.float16) for k, v in w.items()}
    ctx = ExecutionContext({"x": torch.from_numpy(x).to(dev, torch.float16),
                            "r": torch.from_numpy(r).to(dev, torch.float16)})
    d = KernelDispatcher(precision=Precision.FP16)
    d.dispatch(Node("QKVProjection", ["x"], ["q", "k", "v"]), ctx,
               {"Wq": T["Wq"], "bq": T["bq"], "Wk": T["Wk"], "bk": T["bk"], "Wv": T["Wv"], "bv": T["bv"]})
    for n, wk in (("q", "Wq"), ("k", "Wk"), ("v", "Wv")):
        ok, worst = fp16_tol(ctx.get_tensor(n).float().cpu().numpy(), ops.linear(x, w[wk]))
        assert ok, (n, worst)
    d.dispatch(Node("FusedAttentionEpilogue", ["x", "r"], ["e"], {"epsilon": 1e-12}), ctx,
               {"Wo": T["Wo"], "bo": T["bo"], "gamma": T["ln1_g"], "beta": T["ln1_b"]})
    ref_e = ops.add_layernorm(ops.linear(x, w["Wo"], w["bo"]), r, w["ln1_g"], w["ln1_b"], 1e-12)
    ok, worst = fp16_tol(ctx.get_tensor("e").float().cpu().numpy(), ref_e)
    assert ok, worst
    d.dispatch(Node("FusedFFN", ["x"], ["f"], {"epsilon": 1e-12}), ctx,
               {"Wi": T["Wi"], "bi": T["bi"], "Wo2": T["Wo2"], "bo2": T["bo2"],
                "gamma": T["ln2_g"], "beta": T["ln2_b"]})
    u = synthetic.round_f16(ops.bias_gelu(ops.linear(x, w["Wi"]), w["bi"], "erf"))
    ref_f = ops.add_layernorm(ops.linear(u, w["Wo2"], w["bo2"]), x, w["ln2_g"], w["ln2_b"], 1e-12)
    _check(ctx.get_tensor("f").float().cpu().numpy(), ref_f)
    assert d.get_dispatch_stats()["kernel_usage"] == {
        "hip_qkv_projection_fp16": 1, "hip_attention_epilogue_fp16": 1, "hip_ffn_fp16": 1}


def test_torch_compile_transformers_bert(dev):
    """The reference's own caller: torch.compile(transformers.BertModel,
    backend="zenith") (zenith/adapters/pytorch_adapter.py:606-744, with the
    SDPA rewrite of zenith/optimization/fx_patterns.py:81-114). A 12-layer
    model with per-layer LayerNorm parameters and non-zero biases, in fp16
    on the GPU, right-padded batch (transformers passes SDPA a boolean
    [B, 1, S, S] mask and an explicit scale). dynamo captures one graph in
    which every Linear, LayerNorm and SDPA node is a HIP leaf, and the output
    matches transformers' fp32 CPU forward at the encoder bar."""
    import copy

    import torch._dynamo
    import torch.nn.functional as F

    from tests.test_gpu_bert_model import _hf_model, _perturb_hf
    from zenith_amd.hooks import backend, fx_optimizer as O

    nl = 12
    hf = _hf_model(layers=nl, act="gelu", seed=8)
    hf.config._attn_implementation = "sdpa"
    _perturb_hf(hf, seed=8)
    B, S = 4, 128
    rng = np.random.default_rng(9)
    ids = torch.from_numpy(rng.integers(0, 5000, (B, S)).astype(np.int64))
    lens = synthetic.padding_lengths(B, S, seed=9)
    mask = torch.from_numpy((np.arange(S)[None, :] < lens[:, None]).astype(np.int64))
    with torch.no_grad():
        ref = hf(input_ids=ids, attention_mask=mask).last_hidden_state.numpy()
    m16 = copy.deepcopy(hf).half().to(dev).eval()
    torch._dynamo.reset()
    be = backend.register_backend("zenith")
    cm = torch.compile(m16, backend="zenith", dynamic=False)
    with torch.no_grad():
        y = cm(input_ids=ids.to(dev), attention_mask=mask.to(dev)).last_hidden_state
    y = y.float().cpu().numpy()
    assert be.compiled_graphs == 1, be.compiled_graphs
    gm = be.last_graph
    left = [n for n in gm.graph.nodes if n.op == "call_function" and n.target in
            (F.linear, F.layer_norm, F.scaled_dot_product_attention, F.gelu)]
    left += [n for n in gm.graph.nodes if n.op == "call_module"
             and isinstance(gm.get_submodule(n.target), (torch.nn.Linear, torch.nn.LayerNorm))]
    assert not left, [n.format_node() for n in left]
    t = O.replaced_targets(gm)
    assert t.count("hip_linear") + t.count("hip_linear_gelu") == 6 * nl, t
    assert t.count("hip_linear_gelu") == nl and t.count("hip_attention") == nl
    assert t.count("hip_add_layernorm_eps") + t.count("hip_layernorm") == 2 * nl + 1
    rel = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
    worst = float(np.max(np.abs(y - ref) - (2e-2 + 2e-2 * np.abs(ref))))
    print(f"torch.compile(transformers BertModel, backend='zenith'), {nl} layers: "
          f"rel {rel:.3e}, elementwise excess {worst:.3e}")
    assert rel <= 2e-2 and worst <= 0, (rel, worst)
    torch._dynamo.reset()
