"""GPU parity: embedding gather, the fused BERT embedding layer, and the full
BertModel (embeddings + fp16 encoder) loaded from a transformers model and
from a saved checkpoint, vs the CPU oracle and transformers' own forward."""

import numpy as np
import pytest
import torch

from oracle import ops
from tests.conftest import fp16_tol
from zenith_amd import synthetic

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,H", [(torch.float32, 768), (torch.float16, 768), (torch.float32, 30)])
def test_embedding_gather(dev, dtype, H):
    from zenith_amd import _lib as L

    V, n = 1000, 777
    table = torch.from_numpy(synthetic.normal((V, H), tag=1)).to(dev, dtype)
    ids = torch.from_numpy(np.random.default_rng(1).integers(-5, V + 5, n).astype(np.int32)).to(dev)
    out = torch.empty((n, H), dtype=dtype, device=dev)
    L.call("zk_embedding", ids.data_ptr(), table.data_ptr(), out.data_ptr(), n, H, V,
           L.ZK_F32 if dtype == torch.float32 else L.ZK_F16, torch.cuda.current_stream().cuda_stream)
    idn = ids.cpu().numpy()
    ok = (idn >= 0) & (idn < V)
    ref = np.zeros((n, H), np.float32)
    ref[ok] = table.float().cpu().numpy()[idn[ok]]
    np.testing.assert_array_equal(out.float().cpu().numpy(), ref)


def _hf_model(layers=2, act="gelu", seed=0, pooler=False):
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(seed)
    cfg = transformers.BertConfig(hidden_size=768, num_attention_heads=12, intermediate_size=3072,
                                  num_hidden_layers=layers, hidden_act=act, vocab_size=5000,
                                  max_position_embeddings=512, type_vocab_size=2)
    cfg._attn_implementation = "eager"
    return transformers.BertModel(cfg, add_pooling_layer=pooler).eval()


def test_bert_embeddings_vs_oracle(dev):
    from zenith_amd.bert_model import BertModel

    hf = _hf_model(layers=1)
    m = BertModel.from_hf(hf, device=dev)
    B, S = 3, 100
    rng = np.random.default_rng(2)
    ids = rng.integers(0, 5000, (B, S)).astype(np.int32)
    tt = rng.integers(0, 2, (B, S)).astype(np.int32)
    y = m.embed(torch.from_numpy(ids), torch.from_numpy(tt), pos_offset=7).float().cpu().numpy()
    sd = {k: v.detach().numpy() for k, v in hf.state_dict().items()}
    r16 = synthetic.round_f16
    x = (r16(sd["embeddings.word_embeddings.weight"])[ids]
         + r16(sd["embeddings.position_embeddings.weight"])[7:7 + S][None]
         + r16(sd["embeddings.token_type_embeddings.weight"])[tt])
    ref = ops.layernorm(x.reshape(B * S, 768), r16(sd["embeddings.LayerNorm.weight"]),
                        r16(sd["embeddings.LayerNorm.bias"]), 1e-12).reshape(B, S, 768)
    ok, worst = fp16_tol(y, ref)
    assert ok, worst


@pytest.mark.parametrize("act", ["gelu", "gelu_new"])
def test_bert_model_vs_transformers(dev, act, tmp_path):
    """Full model from input_ids with right padding, against transformers'
    fp32 forward; then the same weights through save_pretrained (safetensors)
    and from_pretrained give bit-identical outputs."""
    from zenith_amd.bert_model import BertModel

    hf = _hf_model(layers=2, act=act, seed=1)
    B, S = 4, 128
    rng = np.random.default_rng(3)
    ids = rng.integers(0, 5000, (B, S)).astype(np.int64)
    tt = rng.integers(0, 2, (B, S)).astype(np.int64)
    lens = synthetic.padding_lengths(B, S, seed=3)
    mask = (np.arange(S)[None, :] < lens[:, None]).astype(np.int64)
    with torch.no_grad():
        ref = hf(input_ids=torch.from_numpy(ids), attention_mask=torch.from_numpy(mask),
                 token_type_ids=torch.from_numpy(tt)).last_hidden_state.numpy()
    m = BertModel.from_hf(hf, device=dev)
    y = m(torch.from_numpy(ids), attention_mask=torch.from_numpy(mask),
          token_type_ids=torch.from_numpy(tt)).float().cpu().numpy()
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 2e-2 and np.all(np.abs(y - ref) <= 2e-2 + 2e-2 * np.abs(ref)), rel
    hf.save_pretrained(tmp_path, safe_serialization=True)
    m2 = BertModel.from_pretrained(str(tmp_path), device=dev)
    y2 = m2(torch.from_numpy(ids), attention_mask=torch.from_numpy(mask),
            token_type_ids=torch.from_numpy(tt)).float().cpu().numpy()
    np.testing.assert_array_equal(y2, y)


def test_bert_model_rejects_non_prefix_mask(dev):
    from zenith_amd.bert_model import BertModel

    m = BertModel.from_hf(_hf_model(layers=1), device=dev)
    ids = torch.zeros((1, 8), dtype=torch.int32)
    with pytest.raises(RuntimeError):
        m(ids, attention_mask=torch.tensor([[1, 0, 1, 1, 1, 1, 1, 1]]))


def test_bert_pooler_vs_transformers(dev, tmp_path):
    """pooler_output = tanh(dense(h[:, 0])) against transformers' BertPooler
    on the same model, and through a saved checkpoint; a model without
    pooler weights refuses `pool`."""
    from zenith_amd.bert_model import BertModel

    hf = _hf_model(layers=1, act="gelu", seed=4, pooler=True)
    B, S = 5, 64
    rng = np.random.default_rng(5)
    ids = rng.integers(0, 5000, (B, S)).astype(np.int64)
    with torch.no_grad():
        out = hf(input_ids=torch.from_numpy(ids))
    m = BertModel.from_hf(hf, device=dev)
    h = m(torch.from_numpy(ids))
    p = m.pool(h).float().cpu().numpy()
    ref = out.pooler_output.numpy()
    assert p.shape == (B, 768)
    assert np.all(np.abs(p - ref) <= 2e-2 + 2e-2 * np.abs(ref)), np.abs(p - ref).max()
    # the pooler alone, on the model's own hidden state, vs the oracle
    sd = {k: v.detach().numpy() for k, v in hf.state_dict().items()}
    cls = h[:, 0].float().cpu().numpy()
    r16 = synthetic.round_f16
    ref2 = ops.tanh(ops.matmul_f64(cls, r16(sd["pooler.dense.weight"]).T).astype(np.float32)
                    + r16(sd["pooler.dense.bias"]))
    ok, worst = fp16_tol(p, ref2)
    assert ok, worst
    hf.save_pretrained(tmp_path, safe_serialization=True)
    m2 = BertModel.from_pretrained(str(tmp_path), device=dev)
    np.testing.assert_array_equal(m2.pool(m2(torch.from_numpy(ids))).float().cpu().numpy(), p)
    with pytest.raises(RuntimeError):
        BertModel.from_hf(_hf_model(layers=1), device=dev).pool(h)


def _perturb_hf(hf, seed=42):
    """In place: every LayerNorm gamma ~ 1 + N(0, 0.1), beta ~ N(0, 0.1), the
    query biases ~ N(0, 0.5) and every other Linear bias ~ N(0, 0.05), drawn
    per parameter (the distributions of synthetic.perturb_norms_and_biases),
    instead of transformers' init (gamma 1, beta 0, biases 0 everywhere)."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in hf.named_parameters():
            if name.endswith("LayerNorm.weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            elif name.endswith("LayerNorm.bias"):
                p.copy_(0.1 * torch.randn(p.shape, generator=g))
            elif name.endswith(".bias"):
                std = 0.5 if ".query." in name else 0.05
                p.copy_(std * torch.randn(p.shape, generator=g))
    return hf


def test_bert_model_wired_vs_transformers(dev):
    """12 layers with per-layer LayerNorm parameters and non-zero biases
    (the situation of a trained checkpoint), right-padded batch: the
    encoder's LayerNorm folding and per-head bias interleave against
    transformers' fp32 forward on the same weights, at the encoder bar."""
    from zenith_amd.bert_model import BertModel

    hf = _perturb_hf(_hf_model(layers=12, act="gelu", seed=6), seed=6)
    B, S = 16, 128  # 2048 rows: the folded layers (fewer rows run unfolded)
    rng = np.random.default_rng(7)
    ids = rng.integers(0, 5000, (B, S)).astype(np.int64)
    lens = synthetic.padding_lengths(B, S, seed=7)
    mask = (np.arange(S)[None, :] < lens[:, None]).astype(np.int64)
    with torch.no_grad():
        ref = hf(input_ids=torch.from_numpy(ids),
                 attention_mask=torch.from_numpy(mask)).last_hidden_state.numpy()
    m = BertModel.from_hf(hf, device=dev)
    assert m.encoder.folded(S, B)
    y = m(torch.from_numpy(ids), attention_mask=torch.from_numpy(mask)).float().cpu().numpy()
    rel = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
    worst = float(np.max(np.abs(y - ref) - (2e-2 + 2e-2 * np.abs(ref))))
    print(f"BertModel wired 12 layers vs transformers: rel {rel:.3e}, elementwise excess {worst:.3e}")
    assert rel <= 2e-2 and worst <= 0, (rel, worst)
