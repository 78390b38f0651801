"""BERT encoder on the zenith_amd kernels (fp16 and INT8-FFN variants).

One post-LN layer is seven launches, in the reference encoder's order
(benchmarks/bert_fp16_full.py:96-145, bert_hybrid.py:96-146) but fused:

  1. QKV GEMM + bias            x[M,H] . Wqkv[3H,H]^T         -> qkv[M,3H]
  2. flash attention            reads Q/K/V straight out of qkv by stride
                                (no split/transpose kernels), writes ctx[M,H]
     For sequences of 64 or 128 tokens and head_dim 64, steps 1-2 are one
     launch (zk_qkv_attn_f16): each 256 x 192 GEMM tile is one head of whole
     sequences and runs their attention in its epilogue, so Q, K and V never
     reach HBM (six launches per layer).
  3. out-proj GEMM + bias       ctx . Wo^T                    -> t[M,H]
  4. Add+LayerNorm              LN(t + x)                     -> h1[M,H]
  5. FFN-up GEMM + bias + GELU  h1 . Wi^T                     -> u[M,4H]
  6. FFN-down GEMM + bias       u . Wo2^T                     -> t[M,H]
  7. Add+LayerNorm              LN(t + h1)                    -> out[M,H]

In the INT8-FFN variant step 4 also writes the int8 quantisation of h1,
step 5 is an int8 GEMM whose epilogue dequantises, adds the bias, applies
GELU and re-quantises (int8 out), and step 6 is an int8 GEMM with a dequant
+ bias epilogue. The int8 values equal those of the unfused sequence
(quantise the fp16 tensor), since both quantise the same fp16-rounded value.

With fold_layernorm (the default) the LayerNorms are folded into the GEMMs
that consume them (see _run_folded): four launches per fp16 layer, five
with the INT8 FFN.

All activations live in buffers allocated once per (batch, seq); the whole
forward can be captured into a HIP graph (torch.cuda.CUDAGraph) and replayed,
which removes the ~84 host launches per forward from the critical path.
Weights stay resident in HBM; 12 fp16 layers are ~170 MB.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib as L

F16 = torch.float16

# Rows (batch x seq) below which a forward runs as a small batch (see
# BertEncoder.small_batch). Measured per step at s128 (12 layers, HIP-graph
# replay), folded against small-batch path: b1 0.835 / 0.606 ms, b2 0.924 /
# 0.642, b4 0.945 / 0.757, b8 1.000 / 0.962, b16 1.025 / 1.033.
SPLIT_ROWS = 2048

# Extra elements per row of the fp16 FFN intermediate (FFN-up output,
# FFN-down input) and of the fp16 FFN-down weight. With FFN 3072 an unpadded
# row is 6144 bytes (48 L2 lines): 6528-byte rows measured 29.1 -> 27.3 us for
# the FFN-down GEMM alone and 1.233 -> 1.214 ms per b32 s128 encoder step.
# The int8 intermediate keeps its 3072-byte rows (padded, the INT8-FFN step
# was 3% slower).
FFN_PAD = 192


def to_fragment_order(x: torch.Tensor) -> torch.Tensor:
    """x [R, K] in fragment order, the layout of the *_frag entry points'
    FFN intermediate: for row block rb and k-step ks (E = 8 fp16 or 16 int8
    values per lane, 2 E per k-step; K a multiple of 2 E), 64 lanes x 16
    bytes, lane l holding x[32 rb + l % 32, 2 E ks + E (l // 32) .. +E-1].
    Rows are zero-padded to a multiple of 32; returned flat."""
    R, K = x.shape
    E = 16 // x.element_size()
    Rp = -(-R // 32) * 32
    xp = torch.zeros((Rp, K), dtype=x.dtype, device=x.device)
    xp[:R] = x
    return xp.reshape(Rp // 32, 32, K // (2 * E), 2, E).permute(0, 2, 3, 1, 4).reshape(-1).contiguous()


def from_fragment_order(p: torch.Tensor, R: int, K: int) -> torch.Tensor:
    """The [R, K] matrix held in fragment order by p (inverse of
    to_fragment_order)."""
    E = 16 // p.element_size()
    Rp = -(-R // 32) * 32
    x = p[:Rp * K].reshape(Rp // 32, K // (2 * E), 2, 32, E).permute(0, 3, 1, 2, 4).reshape(Rp, K)
    return x[:R]


def _dev(a: np.ndarray, dtype, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dtype)


def quantize_weight_per_channel(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-output-channel int8 weights: s[n] = max|W[n,:]| / 127,
    q = clamp(round_half_even(W / s[n]), -128, 127) (host-side, once).
    Reference rule: per-channel FakeQuantize (zenith/optimization/qat.py:
    185-270) with the /127 scale of quantization.py:106."""
    w = w.detach().to(torch.float32).cpu()
    amax = w.abs().amax(dim=1)
    s = torch.where(amax > 0, amax / 127.0, torch.ones_like(amax))
    q = torch.clamp(torch.round(w / s[:, None]), -128, 127).to(torch.int8)
    return q, s


def fold_layernorm(w: np.ndarray, b: np.ndarray, gamma: np.ndarray, beta: np.ndarray):
    """LayerNorm(x; gamma, beta) . w^T + b folded into the GEMM on x:
    returns (w' as fp16-rounded float32 [N, K], s [N], c [N]) with
    w'[n, k] = w[n, k] gamma[k], s = column sums of the rounded w', and
    c = beta . w^T + b, so that LN(x) . w^T + b = rstd (x . w'^T - mean s) + c
    (zk_gemm_f16_ln, zk_qkv_attn_f16_ln). w as stored (fp16-rounded)."""
    w = np.asarray(w, np.float32)
    wf = (w * np.asarray(gamma, np.float32)[None, :]).astype(np.float16).astype(np.float32)
    s = wf.astype(np.float64).sum(1).astype(np.float32)
    c = (w.astype(np.float64) @ np.asarray(beta, np.float64) + np.asarray(b, np.float64)).astype(np.float32)
    return wf, s, c


class BertEncoder:
    """12-layer (by default) BERT encoder resident on one GPU.

    layers: list of dicts of float32 numpy arrays with keys
    Wq,bq,Wk,bk,Wv,bv,Wo,bo,ln1_g,ln1_b,Wi,bi,Wo2,bo2,ln2_g,ln2_b
    (torch-Linear layout W[out, in]).
    """

    def __init__(self, layers: list[dict], heads: int = 12, eps: float = 1e-12,
                 gelu: str = "erf", device: str | torch.device = "cuda",
                 fuse_qkv_attention: bool = True, fold_layernorm: bool = True,
                 split_rows: int = SPLIT_ROWS):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("BertEncoder runs on a GPU device")
        L.load()  # fail loudly before any work if the kernels are missing
        self.heads = heads
        self.eps = float(eps)
        self.gelu_epi = L.ZK_EPI_BIAS_GELU_ERF if gelu == "erf" else L.ZK_EPI_BIAS_GELU_TANH
        self.hidden = layers[0]["Wq"].shape[1]
        self.ffn = layers[0]["Wi"].shape[0]
        if self.hidden % heads:
            raise RuntimeError("hidden size must be a multiple of heads")
        self.head_dim = self.hidden // heads
        self.fuse_qkv_attention = bool(fuse_qkv_attention)
        # below this many rows (batch x seq) the layers run unfolded, with
        # split-K GEMMs through a workspace (see _buffers and small_batch)
        self.split_rows = int(split_rows)
        # LayerNorms folded into the GEMMs that consume them (fp16 FFN, erf
        # GELU, hidden size a multiple of 96 up to 1536: the row statistics
        # travel as (mean, M2) of 96-column segments)
        self.fold_ln = (bool(fold_layernorm) and gelu == "erf" and self.hidden % 96 == 0
                        and self.hidden <= 1536)
        # the folded fp16 FFN passes its intermediate in fragment order where
        # it can (see frag_ffn), and so does the fused attention its output;
        # read when the buffers are made
        self.ffn_frag = True
        self.attn_frag = True
        d = self.device
        self.layers = []
        for i, w in enumerate(layers):
            # Q, K, V weights interleaved per head (q_h, k_h, v_h): one GEMM
            # tile of 3 * head_dim columns is one head, for the fused kernel;
            # the unfused attention reads the same layout by stride.
            self.layers.append({
                "Wqkv": _dev(self._per_head(w["Wq"], w["Wk"], w["Wv"]), F16, d),
                "bqkv": _dev(self._per_head(w["bq"], w["bk"], w["bv"]), F16, d),
                "Wo": _dev(w["Wo"], F16, d), "bo": _dev(w["bo"], F16, d),
                "ln1_g": _dev(w["ln1_g"], F16, d), "ln1_b": _dev(w["ln1_b"], F16, d),
                "Wi": _dev(w["Wi"], F16, d), "bi": _dev(w["bi"], F16, d),
                "Wo2": self._padded(_dev(w["Wo2"], F16, d)), "bo2": _dev(w["bo2"], F16, d),
                "ln2_g": _dev(w["ln2_g"], F16, d), "ln2_b": _dev(w["ln2_b"], F16, d),
            })
            if self.fold_ln:
                self.layers[-1].update(self._folded(w, layers[i - 1] if i > 0 else None))
        self.int8 = None
        self._bufs = None
        self._graph = None

    @staticmethod
    def _padded(t: torch.Tensor) -> torch.Tensor:
        """t [rows, FFN] as a view of a [rows, FFN + FFN_PAD] buffer (zero
        padding), so that its row pitch is the FFN intermediate's."""
        full = torch.zeros((t.shape[0], t.shape[1] + FFN_PAD), dtype=t.dtype, device=t.device)
        full[:, :t.shape[1]] = t
        return full[:, :t.shape[1]]

    def _per_head(self, q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
        D = self.head_dim
        parts = []
        for h in range(self.heads):
            parts += [q[h * D:(h + 1) * D], k[h * D:(h + 1) * D], v[h * D:(h + 1) * D]]
        return np.concatenate(parts, 0)

    def _folded(self, w: dict, prev: dict | None) -> dict:
        """LN1 folded into FFN-up, and the previous layer's LN2 into this
        layer's QKV projection (weights, gamma and beta as stored in fp16)."""
        d, r16 = self.device, (lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32))
        f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(d)  # noqa: E731
        wi, si, ci = fold_layernorm(r16(w["Wi"]), r16(w["bi"]), r16(w["ln1_g"]), r16(w["ln1_b"]))
        out = {"Wi_f": _dev(wi, F16, d), "s_i": f32(si), "c_i": f32(ci)}
        if prev is not None:
            wq, sq, cq = fold_layernorm(r16(self._per_head(w["Wq"], w["Wk"], w["Wv"])),
                                        r16(self._per_head(w["bq"], w["bk"], w["bv"])),
                                        r16(prev["ln2_g"]), r16(prev["ln2_b"]))
            out.update({"Wqkv_f": _dev(wq, F16, d), "s_qkv": f32(sq), "c_qkv": f32(cq)})
        return out

    def small_batch(self, B: int | None, S: int) -> bool:
        """Whether B sequences of S tokens (B*S rows) run as a small batch:
        the fused and folded kernels tile 128 or 256 rows at a time, so a few
        sequences leave most CUs idle (b4 s128: 24 to 32 workgroups per
        launch on 256 CUs); below split_rows rows the layers run unfolded,
        with 64x64 GEMM tiles, split-K through a workspace where even those
        are too few, and the separate attention and Add+LayerNorm kernels
        (at least 128 workgroups per launch from four 128-token sequences)."""
        return B is not None and B * S < self.split_rows

    def fused_attention(self, S: int, B: int | None = None) -> bool:
        """Whether sequences of S tokens take the fused QKV + attention
        launch (zk_qkv_attn_f16: S of 64 or 128, head_dim 64; not for a
        small batch of B)."""
        return (self.fuse_qkv_attention and S in (64, 128) and self.head_dim == 64
                and not self.small_batch(B, S))

    def frag_ffn(self, M: int) -> bool:
        """Whether the folded fp16 FFN of M rows passes its intermediate in
        fragment order (zk_gemm_f16_ln_frag, zk_gemm_f16_res_stats_frag; the
        output is the same, bit for bit): wherever zk_gemm_f16_res_stats
        would run the 128x96 tile, i.e. unless M >= 1024 and its 256x192
        tiles number at least 160 (s512 at b32). FFN-up then stores whole
        1 KB blocks instead of 192-byte row pieces (27.4 against 28.4 us at
        b32 s128), and the encoder step is 1.3% faster. The INT8 FFN does the
        same with its int8 intermediate (zk_gemm_i8_requant_frag,
        zk_gemm_i8_res_stats_frag; FFN a multiple of 128)."""
        H = self.hidden
        t192 = -(-M // 256) * (H // 192) if H % 192 == 0 else 0
        return (self.ffn_frag and self.fold_ln and self.ffn % 64 == 0
                and not (M >= 1024 and t192 >= 160))

    def folded(self, S: int, B: int | None = None) -> bool:
        """Whether sequences of S tokens run with the LayerNorms folded into
        the GEMMs. With the INT8 FFN only where the QKV projection and
        attention are one launch: at b32 s128 folding took the INT8-FFN
        encoder from 1.064 to 1.034 ms per step, at s512 from 3.558 to 3.608
        (the residual and statistics epilogue of the 256x192-tile int8
        FFN-down and the LayerNorm-folded 256x256 QKV GEMM cost more than the
        Add+LayerNorm launch they replace)."""
        if self.small_batch(B, S):
            return False
        return self.fold_ln and (self.int8 is None or self.fused_attention(S))

    # ------------------------------------------------------------ INT8 FFN --
    def enable_int8_ffn(self, s_x: list[float], s_h: list[float], layers_fp32: list[dict] | None = None):
        """Switch the FFN to int8 with per-layer activation scales s_x (FFN-up
        input) and s_h (GELU output); weights are quantised per output channel
        from the fp32 masters if given, else from the resident fp16 weights."""
        self.int8 = []
        for i, lw in enumerate(self.layers):
            if layers_fp32 is not None:
                wi = torch.from_numpy(layers_fp32[i]["Wi"])
                wo2 = torch.from_numpy(layers_fp32[i]["Wo2"])
            else:
                wi, wo2 = lw["Wi"], lw["Wo2"]
            qi, si = quantize_weight_per_channel(wi)
            qo, so = quantize_weight_per_channel(wo2)
            self.int8.append({
                "Wi_q": qi.to(self.device), "s_wi": si.to(self.device),
                "Wo2_q": qo.to(self.device), "s_wo2": so.to(self.device),
                "s_x": float(s_x[i]), "s_h": float(s_h[i]),
            })
        self._graph = None

    def disable_int8_ffn(self):
        self.int8 = None
        self._graph = None

    # ------------------------------------------------------------- buffers --
    def _buffers(self, B: int, S: int):
        key = (B, S)
        if self._bufs is not None and self._bufs["key"] == key:
            return self._bufs
        M, H, I, d = B * S, self.hidden, self.ffn, self.device
        self._bufs = {
            "key": key,
            "qkv": torch.empty((M, 3 * H), dtype=F16, device=d),
            "ctx": torch.empty((M, H), dtype=F16, device=d),
            "t": torch.empty((M, H), dtype=F16, device=d),
            "h1": torch.empty((M, H), dtype=F16, device=d),
            "u": torch.empty((M, I + FFN_PAD), dtype=F16, device=d)[:, :I],
            "ping": torch.empty((M, H), dtype=F16, device=d),
            "pong": torch.empty((M, H), dtype=F16, device=d),
            "q_h": torch.empty((M, H), dtype=torch.int8, device=d),
            "q_u": torch.empty((M, I), dtype=torch.int8, device=d),
        }
        # split-K partials of the unfolded GEMMs (zero bytes at large M,
        # where no product is split)
        H3 = 3 * H
        ws = max(int(L.load().zk_gemm_workspace_size(M, n, k, L.ZK_F16))
                 for n, k in ((H3, H), (H, H), (I, H), (H, I)))
        self._bufs["ws"] = torch.empty(ws, dtype=torch.uint8, device=d) if ws else None
        if self.fold_ln:
            f32 = torch.float32
            self._bufs.update({
                # partial (mean, M2) per 96-column segment of h and of h2
                "p1": torch.empty((M, H // 96, 2), dtype=f32, device=d),
                "p2a": torch.empty((M, H // 96, 2), dtype=f32, device=d),
                "p2b": torch.empty((M, H // 96, 2), dtype=f32, device=d),
                # (mean, rstd) per row of h (LN1) and of the layer input (LN2)
                "mr1": torch.empty((M, 2), dtype=f32, device=d),
                "mr2": torch.empty((M, 2), dtype=f32, device=d),
                # the FFN intermediate in fragment order (whole 32-row
                # blocks; the rows past M stay zero)
                "u_frag": (torch.zeros(-(-M // 32) * 32 * I, dtype=F16, device=d)
                           if self.frag_ffn(M) else None),
                "q_u_frag": (torch.zeros(-(-M // 32) * 32 * I, dtype=torch.int8, device=d)
                             if self.frag_ffn(M) and I % 128 == 0 else None),
                # the attention output in fragment order (fp16 layers with
                # the fused QKV + attention launch)
                "ctx_frag": (torch.zeros(-(-M // 32) * 32 * H, dtype=F16, device=d)
                             if self.attn_frag and self.frag_ffn(M) and self.fused_attention(S, B)
                             else None),
            })
        self._graph = None
        return self._bufs

    # ------------------------------------------------------------- forward --
    def _gemm(self, a, w, b, out, epi, residual=None, stream=None, split=True):
        """out = epi(a . w^T + b); small-M products split along K through
        the buffers' workspace (zk_gemm_f16_ws), a fixed-order reduction.
        split=False: no workspace, so the product is not split."""
        M, K = a.shape
        N = w.shape[0]
        ws = self._bufs.get("ws") if self._bufs is not None and split else None
        L.call("zk_gemm_f16_ws", a.data_ptr(), w.data_ptr(), out.data_ptr(), M, N, K,
               a.stride(0), w.stride(0), out.stride(0), 1, L.ZK_F16, b.data_ptr(),
               None if residual is None else residual.data_ptr(),
               0 if residual is None else residual.stride(0), epi,
               None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), stream)

    def _gemm_add_ln(self, a, w, b, res, g, beta, tmp, out, stream):
        """out = LayerNorm(a . w^T + b + res) (zk_gemm_f16_add_ln): where the
        product splits along K, the LayerNorm launch sums the split partials
        itself (one launch fewer); otherwise the product goes through tmp."""
        M, K = a.shape
        N = w.shape[0]
        ws = self._bufs.get("ws") if self._bufs is not None else None
        L.call("zk_gemm_f16_add_ln", a.data_ptr(), w.data_ptr(), b.data_ptr(), res.data_ptr(),
               g.data_ptr(), beta.data_ptr(), tmp.data_ptr(), out.data_ptr(), M, N, K,
               a.stride(0), w.stride(0), self.eps, None if ws is None else ws.data_ptr(),
               0 if ws is None else ws.numel(), stream)

    def _layer(self, i: int, x: torch.Tensor, out: torch.Tensor, lens, B: int, S: int, stream):
        w = self.layers[i]
        bf = self._bufs
        H, D, nh = self.hidden, self.head_dim, self.heads
        M = B * S
        qkv, ctx, t, h1, u = bf["qkv"], bf["ctx"], bf["t"], bf["h1"], bf["u"]
        scale = float(1.0 / np.sqrt(D))
        if self.fused_attention(S, B):
            L.call("zk_qkv_attn_f16", x.data_ptr(), w["Wqkv"].data_ptr(), w["bqkv"].data_ptr(),
                   ctx.data_ptr(), B, S, H, nh, None if lens is None else lens.data_ptr(),
                   scale, stream)
        else:
            self._gemm(x, w["Wqkv"], w["bqkv"], qkv, L.ZK_EPI_BIAS, stream=stream)
            self._attention(qkv, ctx, lens, B, S, stream)
        if self.int8 is None:
            # out-projection + Add+LN1, FFN-up + GELU, FFN-down + Add+LN2
            self._gemm_add_ln(ctx, w["Wo"], w["bo"], x, w["ln1_g"], w["ln1_b"], t, h1, stream)
            # FFN-up whole where it has at least 96 tiles of 64 x 64 (b1: 128 x 3072):
            # its split's reduction launch (with GELU) costs more than the split
            # saves (b1 s128 0.514 -> 0.496 ms per step, b2 and b4 unchanged)
            t64 = -(-M // 64) * -(-self.ffn // 64)
            self._gemm(h1, w["Wi"], w["bi"], u, self.gelu_epi, stream=stream, split=t64 < 96)
            self._gemm_add_ln(u, w["Wo2"], w["bo2"], h1, w["ln2_g"], w["ln2_b"], t, out, stream)
            return
        # INT8 FFN: Add+LN1 also writes the int8 FFN input; FFN-up re-quantises
        # its GELU output in the epilogue (no fp16 intermediate).
        self._gemm(ctx, w["Wo"], w["bo"], t, L.ZK_EPI_BIAS, stream=stream)
        q = self.int8[i]
        qh, qu = bf["q_h"], bf["q_u"]
        L.call("zk_layernorm_q8", t.data_ptr(), x.data_ptr(), w["ln1_g"].data_ptr(),
               w["ln1_b"].data_ptr(), h1.data_ptr(), qh.data_ptr(), M, H, self.eps,
               q["s_x"], stream)
        L.call("zk_gemm_i8_requant", qh.data_ptr(), q["Wi_q"].data_ptr(), qu.data_ptr(), M,
               self.ffn, H, H, H, qu.stride(0), q["s_x"], q["s_wi"].data_ptr(),
               w["bi"].data_ptr(), self.gelu_epi, q["s_h"], stream)
        L.call("zk_gemm_i8", qu.data_ptr(), q["Wo2_q"].data_ptr(), t.data_ptr(), M, H, self.ffn,
               qu.stride(0), q["Wo2_q"].stride(0), H, q["s_h"], q["s_wo2"].data_ptr(),
               w["bo2"].data_ptr(), None, 0, L.ZK_EPI_BIAS, L.ZK_F16, stream)
        L.call("zk_layernorm", t.data_ptr(), h1.data_ptr(), w["ln2_g"].data_ptr(),
               w["ln2_b"].data_ptr(), out.data_ptr(), M, H, self.eps, L.ZK_F16, stream)

    def _run(self, x2: torch.Tensor, lens, B: int, S: int, out: torch.Tensor,
             start: int = 0, stop: int | None = None):
        bf = self._bufs
        stream = torch.cuda.current_stream(self.device).cuda_stream
        stop = len(self.layers) if stop is None else stop
        if self.folded(S, B):
            return self._run_folded(x2, lens, B, S, out, start, stop, stream)
        cur = x2
        for i in range(start, stop):
            dst = out if i == stop - 1 else (bf["ping"] if i % 2 == 0 else bf["pong"])
            self._layer(i, cur, dst, lens, B, S, stream)
            cur = dst
        return out

    def _run_folded(self, x2, lens, B, S, out, start, stop, stream):
        """Layers [start, stop) with the LayerNorms folded into the GEMMs:
        four launches per layer. Each layer keeps its output un-normalised
        (h2 = FFN-down + residual) with per-row partial statistics; the next
        layer's QKV projection applies LN2 through its folded weights and
        its out-projection adds LN2(h2) as the residual on the fly; LN1 goes
        the same way into FFN-up and FFN-down. One LayerNorm kernel at the
        end materialises the last output. With the INT8 FFN, LN1 is
        materialised together with its int8 copy (its LN2 residual applied
        on the fly) and the int8 FFN-down writes h2 with its statistics:
        five launches per layer."""
        bf = self._bufs
        H, D, nh, I = self.hidden, self.head_dim, self.heads, self.ffn
        M, eps = B * S, self.eps
        scale = float(1.0 / np.sqrt(D))
        lp = None if lens is None else lens.data_ptr()
        ctx, qkv, h, u = bf["ctx"], bf["qkv"], bf["h1"], bf["u"]
        p1, mr1, mr2 = bf["p1"], bf["mr1"], bf["mr2"]
        cur, cur_parts = x2, None  # layer input: materialised (first layer) or raw h2
        for i in range(start, stop):
            w = self.layers[i]
            first = i == start
            prev = None if first else self.layers[i - 1]
            h2, p2 = (bf["ping"], bf["p2a"]) if i % 2 == 0 else (bf["pong"], bf["p2b"])
            # 1-2. QKV projection (+ LN2 of the previous layer) and attention
            cf = bf.get("ctx_frag")
            if cf is not None:
                # ctx in fragment order for the out-projection below
                L.call("zk_qkv_attn_f16_frag", cur.data_ptr(),
                       w["Wqkv" if first else "Wqkv_f"].data_ptr(), w["bqkv"].data_ptr(),
                       None if first else cur_parts.data_ptr(), self.eps,
                       None if first else w["s_qkv"].data_ptr(),
                       None if first else w["c_qkv"].data_ptr(),
                       None if first else mr2.data_ptr(), cf.data_ptr(), B, S, H, nh, lp, scale,
                       stream)
            elif self.fused_attention(S, B):
                if first:
                    L.call("zk_qkv_attn_f16", cur.data_ptr(), w["Wqkv"].data_ptr(),
                           w["bqkv"].data_ptr(), ctx.data_ptr(), B, S, H, nh, lp, scale, stream)
                else:
                    L.call("zk_qkv_attn_f16_ln", cur.data_ptr(), w["Wqkv_f"].data_ptr(),
                           cur_parts.data_ptr(), self.eps, w["s_qkv"].data_ptr(),
                           w["c_qkv"].data_ptr(), mr2.data_ptr(), ctx.data_ptr(), B, S, H, nh,
                           lp, scale, stream)
            else:
                if first:
                    self._gemm(cur, w["Wqkv"], w["bqkv"], qkv, L.ZK_EPI_BIAS, stream=stream)
                else:
                    L.call("zk_gemm_f16_ln", cur.data_ptr(), w["Wqkv_f"].data_ptr(), qkv.data_ptr(),
                           M, 3 * H, H, H, H, 3 * H, cur_parts.data_ptr(), self.eps,
                           w["s_qkv"].data_ptr(), w["c_qkv"].data_ptr(), mr2.data_ptr(),
                           L.ZK_EPI_BIAS, stream)
                self._attention(qkv, ctx, lens, B, S, stream)
            if self.int8 is None:
                # 3. out-projection + residual (the input, or LN2(input)) -> h, stats
                if cf is not None:
                    L.call("zk_gemm_f16_res_stats_frag", cf.data_ptr(), w["Wo"].data_ptr(),
                           h.data_ptr(), M, H, H, H, H, w["bo"].data_ptr(), cur.data_ptr(), H,
                           None if first else mr2.data_ptr(),
                           None if first else prev["ln2_g"].data_ptr(),
                           None if first else prev["ln2_b"].data_ptr(), p1.data_ptr(), stream)
                else:
                    L.call("zk_gemm_f16_res_stats", ctx.data_ptr(), w["Wo"].data_ptr(),
                           h.data_ptr(), M, H, H, H, H, H, w["bo"].data_ptr(), cur.data_ptr(), H,
                           None if first else mr2.data_ptr(),
                           None if first else prev["ln2_g"].data_ptr(),
                           None if first else prev["ln2_b"].data_ptr(), p1.data_ptr(), stream)
                uf = bf.get("u_frag")
                if uf is not None:
                    # 4-5. the same, the intermediate in fragment order
                    L.call("zk_gemm_f16_ln_frag", h.data_ptr(), w["Wi_f"].data_ptr(),
                           uf.data_ptr(), M, I, H, H, H, p1.data_ptr(), self.eps,
                           w["s_i"].data_ptr(), w["c_i"].data_ptr(), mr1.data_ptr(), stream)
                    L.call("zk_gemm_f16_res_stats_frag", uf.data_ptr(), w["Wo2"].data_ptr(),
                           h2.data_ptr(), M, H, I, w["Wo2"].stride(0), H, w["bo2"].data_ptr(),
                           h.data_ptr(), H, mr1.data_ptr(), w["ln1_g"].data_ptr(),
                           w["ln1_b"].data_ptr(), p2.data_ptr(), stream)
                else:
                    # 4. FFN-up on LN1(h) + GELU
                    L.call("zk_gemm_f16_ln", h.data_ptr(), w["Wi_f"].data_ptr(), u.data_ptr(), M,
                           I, H, H, H, u.stride(0), p1.data_ptr(), self.eps,
                           w["s_i"].data_ptr(), w["c_i"].data_ptr(), mr1.data_ptr(),
                           L.ZK_EPI_BIAS_GELU_ERF, stream)
                    # 5. FFN-down + LN1(h) -> h2, stats
                    L.call("zk_gemm_f16_res_stats", u.data_ptr(), w["Wo2"].data_ptr(),
                           h2.data_ptr(), M, H, I, u.stride(0), w["Wo2"].stride(0), H,
                           w["bo2"].data_ptr(), h.data_ptr(), H, mr1.data_ptr(),
                           w["ln1_g"].data_ptr(), w["ln1_b"].data_ptr(), p2.data_ptr(), stream)
            else:
                # INT8 FFN (five launches): LN1 is materialised, with its int8
                # copy for FFN-up; LN2 stays folded as in the fp16 layer.
                q, qh, qu, t = self.int8[i], bf["q_h"], bf["q_u"], bf["t"]
                # 3. out-projection + bias -> t
                if cf is not None:
                    L.call("zk_gemm_f16_frag", cf.data_ptr(), w["Wo"].data_ptr(), t.data_ptr(),
                           M, H, H, H, H, w["bo"].data_ptr(), stream)
                else:
                    self._gemm(ctx, w["Wo"], w["bo"], t, L.ZK_EPI_BIAS, stream=stream)
                # 4. h = LN1(t + the input, or + LN2(input) on the fly), and q(h)
                if first:
                    L.call("zk_layernorm_q8", t.data_ptr(), cur.data_ptr(), w["ln1_g"].data_ptr(),
                           w["ln1_b"].data_ptr(), h.data_ptr(), qh.data_ptr(), M, H, self.eps,
                           q["s_x"], stream)
                else:
                    L.call("zk_layernorm_q8_res_ln", t.data_ptr(), cur.data_ptr(), mr2.data_ptr(),
                           prev["ln2_g"].data_ptr(), prev["ln2_b"].data_ptr(),
                           w["ln1_g"].data_ptr(), w["ln1_b"].data_ptr(), h.data_ptr(),
                           qh.data_ptr(), M, H, self.eps, q["s_x"], stream)
                qf = bf.get("q_u_frag")
                if qf is not None:
                    # 5-6. the same, the int8 intermediate in fragment order
                    L.call("zk_gemm_i8_requant_frag", qh.data_ptr(), q["Wi_q"].data_ptr(),
                           qf.data_ptr(), M, I, H, H, H, q["s_x"], q["s_wi"].data_ptr(),
                           w["bi"].data_ptr(), self.gelu_epi, q["s_h"], stream)
                    L.call("zk_gemm_i8_res_stats_frag", qf.data_ptr(), q["Wo2_q"].data_ptr(),
                           h2.data_ptr(), M, H, I, q["Wo2_q"].stride(0), H, q["s_h"],
                           q["s_wo2"].data_ptr(), w["bo2"].data_ptr(), h.data_ptr(), H, None,
                           None, None, p2.data_ptr(), stream)
                else:
                    # 5. FFN-up int8 + bias + GELU, re-quantised
                    L.call("zk_gemm_i8_requant", qh.data_ptr(), q["Wi_q"].data_ptr(),
                           qu.data_ptr(), M, I, H, H, H, qu.stride(0), q["s_x"],
                           q["s_wi"].data_ptr(), w["bi"].data_ptr(), self.gelu_epi, q["s_h"],
                           stream)
                    # 6. FFN-down int8 + bias + h -> h2, stats
                    L.call("zk_gemm_i8_res_stats", qu.data_ptr(), q["Wo2_q"].data_ptr(),
                           h2.data_ptr(), M, H, I, qu.stride(0), q["Wo2_q"].stride(0), H,
                           q["s_h"], q["s_wo2"].data_ptr(), w["bo2"].data_ptr(), h.data_ptr(), H,
                           None, None, None, p2.data_ptr(), stream)
            cur, cur_parts = h2, p2
        w = self.layers[stop - 1]
        L.call("zk_layernorm", cur.data_ptr(), None, w["ln2_g"].data_ptr(), w["ln2_b"].data_ptr(),
               out.data_ptr(), M, H, self.eps, L.ZK_F16, stream)
        return out

    def _attention(self, qkv, ctx, lens, B, S, stream):
        """Attention over the per-head q, k, v column blocks of qkv (head h
        at columns 3 D h + (0, D, 2 D))."""
        H, D, nh = self.hidden, self.head_dim, self.heads
        base = qkv.data_ptr()
        es = qkv.element_size()
        ld = 3 * H
        strides = L.strides_arg([S * ld, 3 * D, ld, S * ld, 3 * D, ld, S * ld, 3 * D, ld,
                                 S * H, D, H])
        L.call("zk_flash_attn_fwd", base, base + D * es, base + 2 * D * es, ctx.data_ptr(),
               B, nh, S, S, D, strides, None if lens is None else lens.data_ptr(),
               float(1.0 / np.sqrt(D)), L.ZK_F16, stream)

    def _check(self, x: torch.Tensor, lens):
        if x.dim() != 3 or x.shape[-1] != self.hidden:
            raise RuntimeError(f"expected hidden states [batch, seq, {self.hidden}]")
        if x.dtype != F16 or x.device != self.device:
            raise RuntimeError("hidden states must be float16 on the encoder's device")
        if lens is not None and (lens.dtype != torch.int32 or lens.numel() != x.shape[0]
                                 or lens.device != self.device):
            raise RuntimeError("lengths must be int32 [batch] on the encoder's device")

    def forward(self, x: torch.Tensor, lengths: torch.Tensor | None = None) -> torch.Tensor:
        """x [B, S, H] fp16 -> [B, S, H] fp16; lengths int32 [B] (key padding)."""
        self._check(x, lengths)
        B, S, H = x.shape
        self._buffers(B, S)
        x2 = x.contiguous().view(B * S, H)
        out = torch.empty((B * S, H), dtype=F16, device=self.device)
        self._run(x2, lengths, B, S, out)
        return out.view(B, S, H)

    __call__ = forward

    def forward_layers(self, x: torch.Tensor, lengths: torch.Tensor | None,
                       start: int, stop: int) -> torch.Tensor:
        """Run layers [start, stop) only (same kernels as forward)."""
        self._check(x, lengths)
        if not 0 <= start < stop <= len(self.layers):
            raise RuntimeError("bad layer range")
        B, S, H = x.shape
        self._buffers(B, S)
        out = torch.empty((B * S, H), dtype=F16, device=self.device)
        self._run(x.contiguous().view(B * S, H), lengths, B, S, out, start, stop)
        return out.view(B, S, H)

    def int8_ffn_tensors(self, layer: int) -> dict:
        """After forward_layers(x, lengths, start, layer + 1) with the INT8 FFN,
        the last layer's FFN tensors as it left them in the work buffers:
        "h1" the FFN input (fp16, LN1's output), "q_h" its int8 copy, "q_u"
        the re-quantised GELU output (int8), and "ffn_out" the FFN-down output
        in fp16: dequantised + bias ("residual": False, unfolded layers), or
        with the residual h1 added as well ("residual": True, folded layers,
        whose next step is the LayerNorm of that sum)."""
        if self.int8 is None or self._bufs is None:
            raise RuntimeError("run forward_layers with the INT8 FFN first")
        B, S = self._bufs["key"]
        bf = self._bufs
        if self.folded(S, B):
            out = bf["ping"] if layer % 2 == 0 else bf["pong"]
        else:
            out = bf["t"]
        return {"h1": bf["h1"], "q_h": bf["q_h"], "q_u": bf["q_u"], "ffn_out": out,
                "residual": self.folded(S, B)}

    # --------------------------------------------------------- HIP graph ----
    def capture(self, B: int, S: int, with_lengths: bool = True):
        """Capture one forward at (B, S) into a HIP graph with static input /
        lengths / output tensors; returns (x_static, lens_static, out_static).
        Fill x_static / lens_static, call replay(), read out_static."""
        self._buffers(B, S)
        self._gx = torch.zeros((B, S, self.hidden), dtype=F16, device=self.device)
        self._gl = torch.full((B,), S, dtype=torch.int32, device=self.device) if with_lengths else None
        self._go = torch.empty((B * S, self.hidden), dtype=F16, device=self.device)
        x2 = self._gx.view(B * S, self.hidden)
        # one eager pass so lazily-initialised state exists before capture
        self._run(x2, self._gl, B, S, self._go)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._run(x2, self._gl, B, S, self._go)
        torch.cuda.synchronize(self.device)
        self._graph = g
        return self._gx, self._gl, self._go.view(B, S, self.hidden)

    def replay(self):
        if self._graph is None:
            raise RuntimeError("capture() first")
        self._graph.replay()
        return self._go.view(*self._gx.shape)
