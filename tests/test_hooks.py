"""Graph hooks on the CPU: FX pattern rewrites (which nodes become HIP
calls), registry selection rules, dispatcher argument marshalling and the
compile-backend gating. No kernel runs here; the GPU side of the same hooks
is tests/test_gpu_hooks.py.

Reference behaviour mirrored: pattern registry and FXOptimizer surface
(tests/python/test_fx_patterns.py:13-203), registry priority / precision
fallback (zenith/runtime/kernel_registry.py:118-153, tested in
tests/test_numerical_accuracy.py:86-117), dispatcher marshalling
(zenith/runtime/dispatcher.py:235-315)."""

import warnings

import pytest
import torch
import torch.fx
import torch.nn.functional as F

from zenith_amd.hooks import backend, fx_optimizer as O, fx_patterns as P
from zenith_amd.hooks.dispatcher import (ExecutionContext, KernelDispatcher, Node,
                                         UnsupportedOperationError)
from zenith_amd.hooks.kernel_registry import KernelRegistry, KernelSpec, Precision


# ------------------------------------------------------------ patterns ----
def test_pattern_registry_surface():
    names = [p.name for p in P.get_all_patterns()]
    for n in ("sdpa_to_flash", "gelu_tanh_to_native", "manual_layernorm_to_native"):
        assert n in names
    for p in P.get_all_patterns():
        assert isinstance(p, P.FXPattern) and callable(p.pattern_fn) and callable(p.replacement_fn)
    assert isinstance(P.is_zenith_cuda_available(), bool)


def test_pattern_functions_compute_their_op():
    """The pattern bodies are the ops they claim (the reference's own
    pattern tests, test_fx_patterns.py:151-203)."""
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(2, 3, 8, 16, generator=g) for _ in range(3))
    torch.testing.assert_close(P.sdpa_pattern(q, k, v), F.scaled_dot_product_attention(q, k, v),
                               rtol=1e-5, atol=1e-6)
    x = torch.randn(4, 64, generator=g)
    torch.testing.assert_close(P.gelu_tanh_pattern(x), F.gelu(x, approximate="tanh"),
                               rtol=1e-5, atol=1e-6)
    w, b = torch.randn(64, generator=g), torch.randn(64, generator=g)
    torch.testing.assert_close(P.layernorm_pattern(x, w, b), F.layer_norm(x, (64,), w, b),
                               rtol=1e-5, atol=1e-5)


class _Manual(torch.nn.Module):
    """Reference-style written-out attention / GELU / LayerNorm."""

    def __init__(self):
        super().__init__()
        self.w = torch.nn.Parameter(torch.randn(64, 32))
        self.b = torch.nn.Parameter(torch.randn(64))
        self.g = torch.nn.Parameter(torch.ones(32))
        self.be = torch.nn.Parameter(torch.zeros(32))

    def forward(self, q, k, v, x, r):
        scale = q.shape[-1] ** -0.5
        a = F.softmax(torch.matmul(q, k.transpose(-2, -1)) * scale, dim=-1)
        o = torch.matmul(a, v)
        h = F.gelu(F.linear(x, self.w, self.b))
        t = 0.5 * x * (1.0 + torch.tanh(0.7978845608028654 * (x + 0.044715 * torch.pow(x, 3))))
        mean = t.mean(dim=-1, keepdim=True)
        var = t.var(dim=-1, keepdim=True, unbiased=False)
        ln = (t - mean) / torch.sqrt(var + 1e-5) * self.g + self.be
        return o, h, ln


class _Modules(torch.nn.Module):
    """Module / functional forms (what real encoders and dynamo graphs hold)."""

    def __init__(self):
        super().__init__()
        self.up = torch.nn.Linear(32, 64)
        self.act = torch.nn.GELU()
        self.ln = torch.nn.LayerNorm(64, eps=1e-12)
        self.proj = torch.nn.Linear(64, 64)
        self.ln2 = torch.nn.LayerNorm(64)

    def forward(self, x, r, q, k, v):
        a = F.scaled_dot_product_attention(q, k, v)
        h = self.ln(self.act(self.up(x)) + r)
        m = F.scaled_dot_product_attention(q, k, v, attn_mask=torch.ones(8, 8, dtype=torch.bool))
        return a, self.ln2(self.proj(h)), F.gelu(h, approximate="tanh"), m


def _opt(mod, **kw):
    gm = torch.fx.symbolic_trace(mod)
    opt = O.FXOptimizer(require_gpu_inputs=False, strict=True, **kw)
    return opt.optimize(gm), opt.get_stats()


def test_reference_patterns_rewrite_to_hip_calls():
    gm, st = _opt(_Manual())
    assert sorted(O.replaced_targets(gm)) == sorted(
        ["hip_flash_attention", "hip_linear_gelu", "hip_gelu_tanh", "hip_layernorm"])
    assert st.patterns_failed == 0
    # nothing of the written-out forms is left
    left = {n.target for n in gm.graph.nodes if n.op == "call_function"}
    assert F.softmax not in left and torch.tanh not in left and torch.sqrt not in left


def test_structural_rewrites_modules_and_functionals():
    gm, st = _opt(_Modules())
    t = O.replaced_targets(gm)
    assert t.count("hip_linear_gelu") == 1          # up + GELU fused
    assert t.count("hip_add_layernorm_eps") == 1    # residual + LN fused
    assert t.count("hip_linear") == 1 and t.count("hip_layernorm") == 1
    assert t.count("hip_gelu_tanh") == 1
    assert t.count("hip_flash_attention") == 1      # masked SDPA left as is
    assert any(n.target is F.scaled_dot_product_attention for n in gm.graph.nodes)
    # eps of the module is carried over
    ln = [n for n in gm.graph.nodes if getattr(n.target, "__name__", "") == "hip_add_layernorm_eps"][0]
    assert ln.args[-1] == 1e-12


def test_group_switches_and_cpu_inputs_skip():
    gm, st = _opt(_Modules(), enable_attention=False, enable_activation=False,
                  enable_normalization=False, enable_linear=False)
    assert O.replaced_targets(gm) == []
    gm = torch.fx.symbolic_trace(_Modules())
    opt = O.FXOptimizer()
    opt.optimize(gm, [torch.zeros(2, 32)])
    assert opt.get_stats().skipped_reason and O.replaced_targets(gm) == []


def test_rewritten_graph_refuses_cpu_tensors():
    """The HIP leaves never fall back to torch: CPU tensors raise."""
    gm, _ = _opt(_Modules())
    args = (torch.randn(4, 32), torch.randn(4, 64), *(torch.randn(1, 2, 8, 64) for _ in range(3)))
    with pytest.raises(RuntimeError):
        gm(*args)


def test_backend_gating():
    b = backend.create_compile_backend(opt_level=1)
    gm = torch.fx.symbolic_trace(_Modules())
    assert b(gm, []) == gm.forward
    b2 = backend.create_compile_backend()  # default level 2 rewrites
    gm2 = torch.fx.symbolic_trace(_Modules())
    fwd = b2(gm2, [])
    assert fwd.__self__ is gm2 and len(O.replaced_targets(gm2)) >= 5


# ------------------------------------------------------------ registry ----
def _spec(name, ops, prec, prio, fn=None, **kw):
    return KernelSpec(name=name, op_types=ops, precision=prec, kernel_fn=fn or (lambda *a: name),
                      priority=prio, **kw)


def test_registry_priority_and_precision_fallback():
    reg = KernelRegistry()
    reg.register(_spec("low", ["Linear"], Precision.FP32, 1))
    reg.register(_spec("high", ["Linear"], Precision.FP32, 25))
    reg.register(_spec("mid16", ["Linear"], Precision.FP16, 10))
    assert reg.get_kernel("Linear", Precision.FP32).name == "high"
    assert reg.get_kernel("Linear", Precision.FP16).name == "mid16"
    assert reg.get_kernel("Linear", Precision.BF16).name == "high"  # falls back to FP32
    assert reg.get_kernel("Conv", Precision.FP32) is None
    assert reg.is_supported("Linear", Precision.FP16) and not reg.is_supported("Linear", Precision.INT8)
    assert reg.get_kernel("Linear", Precision.FP32).function is reg.get_kernel("Linear", Precision.FP32).kernel_fn


def test_registry_constraints():
    reg = KernelRegistry()
    reg.register(_spec("small", ["Attention"], Precision.FP16, 30, input_constraints={"max_seq_len": 128}))
    reg.register(_spec("any", ["Attention"], Precision.FP16, 5))
    assert reg.get_kernel("Attention", Precision.FP16, [(2, 128, 64)]).name == "small"
    assert reg.get_kernel("Attention", Precision.FP16, [(2, 512, 64)]).name == "any"


def test_hip_registry_needs_the_library(tmp_path, monkeypatch):
    """initialize() registers only HIP kernels; every fused op type the graph
    passes emit has one."""
    reg = KernelRegistry()
    reg.initialize()
    for op in ("Linear", "Gemm", "MatMul", "LayerNorm", "FusedAddLayerNorm", "AddLayerNorm",
               "FusedBiasGeLU", "LinearGelu", "QKVProjection", "FlashAttention", "Attention",
               "FusedAttentionEpilogue", "FusedFFN", "Gelu", "Relu"):
        k = reg.get_kernel(op, Precision.FP16)
        assert k is not None and k.priority == 25 and k.name.startswith("hip_"), op
    assert reg.get_kernel("Linear", Precision.INT8).name.startswith("hip_qlinear")
    assert reg.get_kernel("LayerNormAdd", Precision.FP32).name.startswith("hip_layernorm_add")


_FUSED_OPS = ("Linear", "Gemm", "MatMul", "LayerNorm", "FusedAddLayerNorm", "AddLayerNorm",
              "LayerNormAdd", "FusedBiasGeLU", "LinearGelu", "QKVProjection", "FlashAttention",
              "Attention", "FusedAttentionEpilogue", "FusedFFN", "Gelu", "Relu")


def test_binding_into_a_foreign_registry():
    """register_hip_kernels on a registry whose Precision is a different Enum
    class (as the reference's is): get_kernel must find the HIP specs at
    FP32, FP16 and INT8, fused op types included. Before the specs were built
    from the registry's own types, every lookup here returned None."""
    from tests import _stand_in_registry as ref
    from zenith_amd.hooks.kernels import register_hip_kernels

    assert ref.Precision is not Precision and ref.Precision.FP16 != Precision.FP16
    reg = ref.KernelRegistry()
    assert register_hip_kernels(reg) > 0
    for prec in (ref.Precision.FP32, ref.Precision.FP16):
        for op in _FUSED_OPS:
            k = reg.get_kernel(op, prec)
            assert k is not None and k.name.startswith("hip_"), (op, prec)
            assert isinstance(k, ref.KernelSpec) and k.precision is prec and k.priority == 25
    k8 = reg.get_kernel("Linear", ref.Precision.INT8)
    assert k8.name.startswith("hip_qlinear") and k8.precision is ref.Precision.INT8
    # BF16 has no HIP spec: the reference rule falls back to FP32
    assert reg.get_kernel("Linear", ref.Precision.BF16).precision is ref.Precision.FP32


def test_binding_with_explicit_types():
    """Explicit spec_cls / precision_enum win over the registry's module; a
    precision the enum lacks is skipped."""
    import enum
    from tests import _stand_in_registry as ref
    from zenith_amd.hooks.kernels import register_hip_kernels

    P2 = enum.Enum("P2", {"FP32": "fp32", "FP16": "fp16"})
    reg = ref.KernelRegistry()
    register_hip_kernels(reg, spec_cls=ref.KernelSpec, precision_enum=P2)
    assert reg.get_kernel("Linear", P2.FP16).precision is P2.FP16
    assert not any(k.name.startswith("hip_qlinear") for k in reg._kernels["Linear"])


def test_register_backend_replaces_an_existing_name():
    """The reference's `import zenith` registers "zenith" first; ours must
    take the name over (or refuse loudly), never keep the other one."""
    from torch._dynamo.backends import registry as R

    name = "zenith_amd_test_backend"

    def other(gm, example_inputs):
        return gm.forward

    R._COMPILER_FNS.pop(name, None)
    R._BACKENDS.pop(name, None)
    R.register_backend(compiler_fn=other, name=name)
    try:
        with pytest.raises(RuntimeError):
            backend.register_backend(name=name, replace=False)
        assert R.lookup_backend(name) is other
        with pytest.warns(RuntimeWarning, match="replacing"):
            ours = backend.register_backend(name=name)
        assert R.lookup_backend(name) is ours and ours is not other
        with warnings.catch_warnings():
            warnings.simplefilter("error")  # replacing our own registration is silent
            ours2 = backend.register_backend(name=name)
        assert R.lookup_backend(name) is ours2
    finally:
        R._COMPILER_FNS.pop(name, None)
        R._BACKENDS.pop(name, None)


# ---------------------------------------------------------- dispatcher ----
class _Rec:
    def __init__(self):
        self.calls = []

    def __call__(self, name):
        def fn(*args, **kw):
            self.calls.append((name, args, kw))
            return name
        return fn


def _disp(rec, prec=Precision.FP32):
    reg = KernelRegistry()
    for op in ("Linear", "MatMul", "LayerNorm", "FusedAddLayerNorm", "GELU", "FusedBiasGeLU",
               "Attention", "FlashAttention", "QKVProjection", "FusedFFN", "LinearGelu",
               "LayerNormAdd"):
        reg.register(_spec(op, [op], prec, 25, fn=rec(op)))
    return KernelDispatcher(registry=reg, precision=prec)


def test_dispatcher_linear_layouts():
    rec = _Rec()
    d = _disp(rec)
    x, W, B, b = torch.zeros(2, 3), torch.zeros(4, 3), torch.zeros(3, 4), torch.zeros(4)
    ctx = ExecutionContext({"x": x, "y": torch.zeros(3, 5)})
    d.dispatch(Node("Linear", ["x"], ["o1"]), ctx, {"weight": W, "bias": b})
    d.dispatch(Node("Gemm", ["x"], ["o2"], {"transB": 1}), ctx, {"B": W, "C": b})
    d.dispatch(Node("Gemm", ["x"], ["o3"]), ctx, {"B": B, "C": b})
    d.dispatch(Node("MatMul", ["x"], ["o4"]), ctx, {"B": B})
    d.dispatch(Node("MatMul", ["x", "y"], ["o5"]), ctx)
    shapes = [(c[0], tuple(c[1][1].shape)) for c in rec.calls]
    # every weighted form reaches the kernel as W[N, K]; two activations stay A . B
    assert shapes == [("Linear", (4, 3)), ("Linear", (4, 3)), ("Linear", (4, 3)),
                      ("Linear", (4, 3)), ("MatMul", (3, 5))]
    assert ctx.get_tensor("o1") == "Linear" and d.get_dispatch_stats()["total_dispatches"] == 5


def test_dispatcher_fused_ops_and_eps():
    rec = _Rec()
    d = _disp(rec, Precision.FP16)
    t = torch.zeros(2, 4)
    ctx = ExecutionContext({"a": t, "r": t, "q": t, "k": t, "v": t, "lens": torch.zeros(2)})
    d.dispatch(Node("LayerNormalization", ["a"], ["o"], {"epsilon": 1e-12}), ctx,
               {"gamma": t[0], "beta": t[0]})
    d.dispatch(Node("AddLayerNorm", ["a", "r"], ["o"]), ctx, {"gamma": t[0], "beta": t[0]})
    d.dispatch(Node("Gelu", ["a"], ["o"], {"approximate": "none"}), ctx)
    d.dispatch(Node("FlashAttention", ["q", "k", "v", "lens"], ["o"], {"scale": 0.125}), ctx)
    d.dispatch(Node("QKVProjection", ["a"], ["q2", "k2", "v2"]), ctx,
               {"Wq": t, "bq": t[0], "Wk": t, "bk": t[0], "Wv": t, "bv": t[0]})
    names = [c[0] for c in rec.calls]
    assert names == ["LayerNorm", "FusedAddLayerNorm", "GELU", "FlashAttention", "QKVProjection"]
    assert rec.calls[0][1][3] == 1e-12 and rec.calls[1][1][4] == 1e-5
    assert rec.calls[2][1][1] == "none"
    assert rec.calls[3][2] == {"key_padding_lengths": ctx.get_tensor("lens"), "scale": 0.125}


def test_dispatcher_layernorm_add_marshalling():
    """LayerNormAdd reaches fn(x, residual, gamma, beta, eps) from both node
    forms: (x, residual) + affine weights, and the four LayerNormalization ->
    Add inputs (x, scale, B, residual)."""
    rec = _Rec()
    d = _disp(rec)
    x, r, g, b = (torch.full((2, 4), float(i)) for i in range(4))
    ctx = ExecutionContext({"x": x, "r": r, "g": g[0], "b": b[0]})
    d.dispatch(Node("LayerNormAdd", ["x", "r"], ["o"], {"epsilon": 1e-12}), ctx,
               {"weight": g[0], "bias": b[0]})
    d.dispatch(Node("FusedLayerNormAdd", ["x", "g", "b", "r"], ["o"]), ctx)
    for name, args, _ in rec.calls:
        assert name == "LayerNormAdd"
        assert args[0] is x and args[1] is r
        assert torch.equal(args[2], g[0]) and torch.equal(args[3], b[0])
    assert rec.calls[0][1][4] == 1e-12 and rec.calls[1][1][4] == 1e-5


def test_dispatcher_unsupported():
    d = _disp(_Rec())
    with pytest.raises(UnsupportedOperationError):
        d.dispatch(Node("Conv", ["a"], ["o"]), ExecutionContext({"a": torch.zeros(1)}))


# ------------------------------------------------------ masked attention ----
class _MaskedSDPA(torch.nn.Module):
    def forward(self, q, k, v, mask):
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)


@pytest.mark.parametrize("mask_dtype,rewritten", [(torch.bool, True), (torch.float32, False)])
def test_sdpa_with_mask_rewrites_only_boolean_masks(mask_dtype, rewritten):
    """With shape metadata on the graph (as torch.compile graphs carry), an
    SDPA call with a boolean mask becomes the masked HIP attention leaf, the
    mask passed through; an additive float mask stays with torch."""
    from torch.fx.passes.shape_prop import ShapeProp

    gm = torch.fx.symbolic_trace(_MaskedSDPA())
    q = torch.randn(2, 3, 8, 16)
    mask = torch.ones(2, 1, 8, 8, dtype=mask_dtype)
    ShapeProp(gm).propagate(q, q, q, mask)
    opt = O.FXOptimizer(require_gpu_inputs=False)
    gm = opt.optimize(gm, [q, q, q, mask])
    calls = [n for n in gm.graph.nodes if n.op == "call_function"]
    hip = [n for n in calls if n.target is P.hip_attention]
    assert bool(hip) == rewritten
    if rewritten:
        assert hip[0].args[4].op == "placeholder" and hip[0].args[4].name == "mask"
        assert not any(n.target is F.scaled_dot_product_attention for n in calls)


def test_sdpa_mask_of_unknown_dtype_is_left_alone():
    gm = torch.fx.symbolic_trace(_MaskedSDPA())  # no shape metadata
    gm = O.FXOptimizer(require_gpu_inputs=False).optimize(gm, [])
    assert not any(n.op == "call_function" and n.target is P.hip_attention for n in gm.graph.nodes)


class _LeafContracts:
    """CPU stand-in for the zenith_cuda functions the FX leaves call: the
    same argument contracts as zenith_amd/zenith_cuda.py (2-D rows and an
    equal-shaped residual for add_layernorm, [N, K] weights for linear,
    4-D Q/K/V and a boolean mask that broadcasts for flash_attention), the
    arithmetic done by torch on the CPU, so that a rewritten graph can run
    here and be compared with the graph it replaced."""

    @staticmethod
    def add_layernorm(input, residual, gamma, beta, eps=1e-5):
        assert input.dim() == 2, "Input must be 2D [batch, hidden]"
        assert residual is None or residual.shape == input.shape, "residual must match input"
        assert gamma.numel() == beta.numel() == input.shape[1]
        x = input if residual is None else input + residual
        return F.layer_norm(x, (x.shape[1],), gamma, beta, eps)

    @classmethod
    def layernorm(cls, input, gamma, beta, eps=1e-5):
        return cls.add_layernorm(input, None, gamma, beta, eps)

    @staticmethod
    def linear(x, weight, bias=None, activation=None, residual=None):
        assert weight.dim() == 2 and x.shape[-1] == weight.shape[1]
        y = F.linear(x, weight, bias)
        return F.gelu(y) if activation == "gelu" else y

    @staticmethod
    def gelu(x, approximate="tanh"):
        return F.gelu(x, approximate=approximate)

    @staticmethod
    def flash_attention(Q, K, V, key_padding_lengths=None, scale=None, attn_mask=None):
        assert Q.dim() == K.dim() == V.dim() == 4 and K.shape == V.shape
        assert Q.shape[-1] <= 128
        if attn_mask is not None:
            assert attn_mask.dtype == torch.bool
            torch.broadcast_shapes(attn_mask.shape, (*Q.shape[:3], K.shape[2]))
        return F.scaled_dot_product_attention(Q, K, V, attn_mask=attn_mask, scale=scale)


def test_transformers_bert_graph_rewritten_to_hip_leaves(monkeypatch):
    """What torch.compile hands the backend for a real transformers BertModel
    (SDPA attention, right-padded batch: a boolean [B, 1, S, S] mask and an
    explicit scale) is rewritten so that every Linear, LayerNorm and SDPA node
    is a HIP leaf; run on the CPU through stand-ins that hold the leaves'
    argument contracts, the rewritten graph gives the original graph's
    output. (The embeddings' Add broadcasts a [1, S, H] position term, so it
    stays a torch add in front of a plain LayerNorm leaf.)"""
    import copy

    transformers = pytest.importorskip("transformers")
    import torch._dynamo

    monkeypatch.setattr(P, "zenith_cuda", _LeafContracts)
    torch.manual_seed(0)
    nl = 2
    cfg = transformers.BertConfig(hidden_size=768, num_attention_heads=12, intermediate_size=3072,
                                  num_hidden_layers=nl, hidden_act="gelu", vocab_size=1000,
                                  max_position_embeddings=128)
    cfg._attn_implementation = "sdpa"
    hf = transformers.BertModel(cfg, add_pooling_layer=False).eval()
    with torch.no_grad():
        for name, p in hf.named_parameters():  # non-trivial LayerNorms and biases
            if name.endswith("LayerNorm.weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape))
            elif name.endswith(".bias"):
                p.copy_(0.1 * torch.randn(p.shape))
    seen = []

    def recording_backend(gm, example_inputs):
        opt = O.FXOptimizer(require_gpu_inputs=False, strict=True)
        new = opt.optimize(copy.deepcopy(gm), example_inputs)
        with torch.no_grad():
            seen.append((new, gm(*example_inputs), new(*example_inputs)))
        return gm.forward

    ids = torch.randint(0, 1000, (2, 16))
    mask = torch.ones(2, 16, dtype=torch.long)
    mask[1, 9:] = 0
    torch._dynamo.reset()
    try:
        with torch.no_grad():
            torch.compile(hf, backend=recording_backend, dynamic=False)(input_ids=ids,
                                                                         attention_mask=mask)
    finally:
        torch._dynamo.reset()
    assert len(seen) == 1
    gm, want, got = seen[0]
    left = [n.format_node() for n in gm.graph.nodes if n.op == "call_function" and n.target in
            (F.linear, F.layer_norm, F.scaled_dot_product_attention, F.gelu)]
    assert not left, left
    t = O.replaced_targets(gm)
    assert t.count("hip_linear") + t.count("hip_linear_gelu") == 6 * nl
    assert t.count("hip_linear_gelu") == nl and t.count("hip_attention") == nl
    assert t.count("hip_add_layernorm_eps") == 2 * nl and t.count("hip_layernorm") == 1
    want = want[0] if isinstance(want, (tuple, list)) else want
    got = got[0] if isinstance(got, (tuple, list)) else got
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-4)
