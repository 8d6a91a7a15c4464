"""GPU parity of the ModernBERT (Laya) encoder path against the CPU oracle (the reference runs
ModernBERT through candle in fp32; the oracle follows the public definition it implements and
is pinned by the golden vectors of tests/golden/modernbert in tests/test_oracle.py).

Tolerances (stated per test): fp32 kernels 1e-4 relative (max error over max magnitude);
16-bit attention 2e-2 (bf16) / 4e-3 (fp16); fp32 encoder hidden states 1e-4 absolute
against the oracle (unit-scale LayerNorm outputs).
"""
import numpy as np
import pytest
import torch

from huncho_amd import abi
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SEED = 31337


@pytest.fixture(scope="module")
def ctx():
    from huncho_amd.ops import context_for_torch

    c = context_for_torch(0)
    yield c
    c.close()


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _round(x, dtype):
    x = np.asarray(x, np.float32)
    if dtype == torch.bfloat16:
        return O.round_bf16(x)
    if dtype == torch.float16:
        return x.astype(np.float16).astype(np.float32)
    return x


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("half_window", [-1, 8, 64])
def test_bidir_attention_varlen(ctx, dtype, half_window):
    """Ragged lengths (1 .. 300, crossing the 64-key tiles and 128-query blocks), 3 heads of
    64, q/k/v read as views of fused [tokens][3][heads][64] rows; global and local windows."""
    from huncho_amd.ops import bidir_attention

    lengths = [1, 5, 63, 64, 65, 130, 300]
    heads = 3
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    n = int(cu[-1])
    qkv = _round(abi.synth_normal(SEED, 10 + (half_window % 97), n * 3 * heads * 64), dtype).reshape(n, 3, heads, 64)
    q, k, v = (np.ascontiguousarray(qkv[:, i]) for i in range(3))
    ref = O.bidir_attention(q, k, v, cu, half_window)
    dev = torch.from_numpy(qkv).to(dtype).cuda()
    out = bidir_attention(ctx, dev[:, 0], dev[:, 1], dev[:, 2], torch.from_numpy(cu).cuda(), max(lengths),
                          half_window)
    torch.cuda.synchronize()
    assert ctx.take_faults() == 0
    err = rel_err(out.float().cpu().numpy(), ref)
    tol = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 4e-3}[dtype]
    print(f"bidir attention {dtype} window {half_window}: {err:.2e}")
    assert err < tol, err


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mean_pool_head(ctx, dtype):
    """Rows of 1, 31, 32, 33 and 700 tokens (fewer, equal and more rows than the 32 partial
    sums): logits against a float64 mean and head on the same values, 1e-5 relative."""
    from huncho_amd.ops import mean_pool_head

    lengths, width, n_out = [1, 31, 32, 33, 700], 768, 4
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    n = int(cu[-1])
    x = _round(abi.synth_normal(SEED, 40, n * width), dtype).reshape(n, width)
    w = _round(abi.synth_normal(SEED, 41, n_out * width, 0.0, 0.05), dtype).reshape(n_out, width)
    b = abi.synth_normal(SEED, 42, n_out)
    got = mean_pool_head(ctx, torch.from_numpy(x).to(dtype).cuda(), torch.from_numpy(cu).cuda(),
                         torch.from_numpy(w).to(dtype).cuda(), torch.from_numpy(b).cuda())
    torch.cuda.synchronize()
    assert ctx.take_faults() == 0
    ref = np.stack([w.astype(np.float64) @ x[cu[s]:cu[s + 1]].astype(np.float64).mean(0) + b for s in range(len(lengths))])
    e = rel_err(got.cpu().numpy(), ref)
    print(f"mean pool head {dtype}: {e:.2e}")
    assert e < 1e-5, e


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("width", [768, 100])
def test_layer_norm(ctx, dtype, width):
    """Widths that take the 16-byte vector path (768) and the scalar path (100)."""
    from huncho_amd.ops import layer_norm

    x = _round(abi.synth_normal(SEED, 40, 37 * width, 0.3, 2.0), dtype).reshape(37, width)
    w = O.round_bf16(abi.synth_normal(SEED, 41, width, 1.0, 0.1))
    y = layer_norm(ctx, torch.from_numpy(x).to(dtype).cuda(), torch.from_numpy(w).cuda(), 1e-5)
    ref = O.layer_norm(x, w, 1e-5)
    err = rel_err(y.float().cpu().numpy(), ref)
    assert err < (1e-5 if dtype == torch.float32 else 1e-2), err


def _laya_from_oracle(cfg, n_out=0, max_context=512):
    from huncho_amd.laya import LayaShape

    return LayaShape(hidden=cfg.hidden_size, n_layers=cfg.num_hidden_layers, n_heads=cfg.num_attention_heads,
                     intermediate=cfg.intermediate_size, vocab=cfg.vocab_size, eps=cfg.layer_norm_eps,
                     global_every=cfg.global_attn_every_n_layers, local_window=cfg.local_attention,
                     global_theta=cfg.global_rope_theta, local_theta=cfg.local_rope_theta, max_context=max_context,
                     n_out=n_out)


def _bert64_weights(seed, H=128, L=4, I=192, V=500):
    names = {"model.embeddings.tok_embeddings.weight": (V, H), "model.embeddings.norm.weight": (H,),
             "model.final_norm.weight": (H,), "head.weight": (4, H)}
    for l in range(L):
        p = f"model.layers.{l}."
        names.update({p + "attn_norm.weight": (H,), p + "attn.Wqkv.weight": (3 * H, H), p + "attn.Wo.weight": (H, H),
                      p + "mlp_norm.weight": (H,), p + "mlp.Wi.weight": (2 * I, H), p + "mlp.Wo.weight": (H, I)})
    w = {}
    for idx, name in enumerate(sorted(names)):
        mean = 1.0 if name.endswith("norm.weight") else 0.0
        std = 0.5 if name.endswith("mlp.Wi.weight") else 0.1
        w[name] = O.round_bf16(O.normal(seed, 900 + idx, names[name], mean, std))
    cfg = O.BertConfig(hidden_size=H, num_hidden_layers=L, num_attention_heads=H // 64, intermediate_size=I,
                       vocab_size=V, global_attn_every_n_layers=3, local_attention=32, global_rope_theta=160000.0,
                       local_rope_theta=10000.0)
    return cfg, w


def _oracle_logits(hidden_rows, head_w):
    return np.stack([head_w.astype(np.float64) @ h.astype(np.float64).mean(0) for h in hidden_rows]).astype(np.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_modernbert_64_matches_oracle(ctx, dtype):
    """A 4-layer encoder with head dim 64 (layers 0 and 3 global, 1 and 2 local with window
    32), ragged rows of 1, 40, 129 and 300 tokens: fp32 hidden states within 1e-4 absolute of
    the oracle's fp32 forward and mean-pooled logits within 1e-4 relative; bf16 hidden states
    within twice the oracle's own bf16-vs-fp32 difference of both oracle flows."""
    from huncho_amd.laya import LayaModel

    cfg, w = _bert64_weights(SEED)
    shape = _laya_from_oracle(cfg, n_out=4)
    rows = [abi.synth_uniform_int(SEED, 950 + i, L, 0, cfg.vocab_size - 1).tolist() for i, L in enumerate([1, 40, 129, 300])]
    model = LayaModel(ctx, shape, w, dtype)
    logits, hs = model.forward_batch(rows, want_hidden=True)
    model.close()
    ref32 = O.BertModel(cfg, w).forward(rows)
    err_h = max(float(np.abs(a - b).max()) for a, b in zip(hs, ref32))
    err_l = rel_err(logits, _oracle_logits(ref32, w["head.weight"]))
    if dtype == torch.float32:
        print(f"ModernBERT-64 fp32: hidden {err_h:.2e} abs, logits {err_l:.2e} rel")
        assert err_h < 1e-4 and err_l < 1e-4, (err_h, err_l)
    else:
        ref16 = O.BertModel(cfg, w, bf16=True).forward(rows)
        err16 = max(float(np.abs(a - b).max()) for a, b in zip(hs, ref16))
        noise = max(float(np.abs(a - b).max()) for a, b in zip(ref16, ref32))
        print(f"ModernBERT-64 bf16: hidden vs oracle bf16 {err16:.2e}, vs fp32 {err_h:.2e} "
              f"(oracle bf16 vs fp32 {noise:.2e}); logits vs fp32 {err_l:.2e} rel")
        assert err16 < 2 * noise and err_h < 2 * noise, (err16, err_h, noise)


def test_laya_shaped_bf16(ctx):
    """The ModernBERT-base shape (hidden 768, 22 layers, 12 heads, GeGLU 1152, vocab 50368,
    local window 128, thetas 160000 / 10000) with seeded bf16 weights, rows of 200, 37 and 513
    tokens: mean-pooled logits against the oracle's bf16 and fp32 flows, inside the bf16
    rounding envelope (5e-2 relative)."""
    from huncho_amd.laya import LayaModel, LayaShape, synthetic_weights

    shape = LayaShape()
    w = synthetic_weights(shape, SEED)
    rows = [abi.synth_uniform_int(SEED, 960 + i, L, 0, shape.vocab - 1).tolist() for i, L in enumerate([200, 37, 513])]
    model = LayaModel(ctx, shape, w, torch.bfloat16)
    logits, _ = model.forward_batch(rows)
    model.close()
    f = {k: O.bf16_to_f32(v).reshape(v.shape) for k, v in w.items()}
    cfg = O.BertConfig(hidden_size=768, num_hidden_layers=22, num_attention_heads=12, intermediate_size=1152,
                       vocab_size=shape.vocab, global_attn_every_n_layers=3, local_attention=128,
                       global_rope_theta=160000.0, local_rope_theta=10000.0)
    ref16 = _oracle_logits(O.BertModel(cfg, f, bf16=True).forward(rows), f["head.weight"])
    ref32 = _oracle_logits(O.BertModel(cfg, f, bf16=False).forward(rows), f["head.weight"])
    e16, e32, noise = rel_err(logits, ref16), rel_err(logits, ref32), rel_err(ref16, ref32)
    print(f"Laya-shaped bf16 logits: vs oracle bf16 {e16:.2e}, vs fp32 {e32:.2e} (oracle bf16 vs fp32 {noise:.2e})")
    assert e16 < 5e-2 and e32 < 5e-2, (e16, e32, noise)


def test_laya_rejects_bad_batches(ctx):
    from huncho_amd.laya import LayaModel

    cfg, w = _bert64_weights(SEED + 1, L=1)
    model = LayaModel(ctx, _laya_from_oracle(cfg, n_out=4), w, torch.bfloat16)
    with pytest.raises(ValueError):
        model.forward_batch([[1, 2], []])
    with pytest.raises(ValueError):
        model.forward_batch([[1, 2, cfg.vocab_size]])
    with pytest.raises(ValueError):
        model.forward_batch([[1]] * 65)
    model.close()
