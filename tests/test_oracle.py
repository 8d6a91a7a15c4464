"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Each check is chosen so a plausible mistake in the oracle fails it:
  * the reference's golden vectors (tiny Kev, kev_reference.rs:61-87 gates) pin the composed
    forward: embedding, GDN conv/prep/recurrence/gated norm, gated GQA attention with
    partial RoPE, MLP, final norm, pointer head and calibration;
  * planted mistakes (no LoRA merge, plain instead of 1+w norm weights, swapped layer
    types) must break the golden match, so the golden is sensitive to them;
  * invariants and closed forms from the reference's own unit tests: delta-rule split
    continuation and special cases (delta_cpu.rs:203-247), paged == dense attention for any
    page permutation and page size (kv_pages.rs:388-630), future-value poisoning, conv
    tap order (conv_cpu.rs:92-140), calibration semantics (calibration.rs:315-430);
  * ModernBERT (no reference golden vectors exist): vectors from an independent
    implementation of the public definition (tests/golden/make_modernbert_vectors.py) on the
    reference's tiny_modernbert checkpoint and a seeded 4-layer model, plus planted
    mistakes (window off by one, tanh GELU, swapped RoPE thetas, missing attention norm).
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


@pytest.fixture(scope="module")
def tiny(golden_dir):
    return O.load_tiny_kev(golden_dir / "tiny_kev")


def _golden_errors(cfg, weights, head, golden):
    m = O.QwenModel(cfg, weights, bf16=False)
    worst_l = worst_p = 0.0
    for case in golden["cases"]:
        for row in case["rows"]:
            h = m.forward(row["tokens"])
            s = O.pointer_head(h, row["positions"], head)
            p = O.calibrate(s, head["temperature"])
            worst_l = max(worst_l, float(np.abs(s - np.float32(row["raw_logits"])).max()))
            worst_p = max(worst_p, float(np.abs(p - np.float32(row["probabilities"])).max()))
    return worst_l, worst_p, m


def test_tiny_kev_golden_fp32(tiny):
    cfg, weights, head, golden = tiny
    worst_l, worst_p, m = _golden_errors(cfg, weights, head, golden)
    assert worst_l < 2e-4, worst_l
    assert worst_p < 2e-5, worst_p
    # short row (kev_reference.rs:75-87): a 2-token row used to underflow the conv
    h = m.forward([1, 2])
    s = O.pointer_head(h, [0], head)
    assert abs(float(s[0]) - golden["short_logits"][0]) < 2e-4


def test_tiny_kev_metadata(tiny):
    cfg, _, head, _ = tiny
    assert abs(head["temperature"] - 2.40605) < 1e-5
    assert cfg.rotary_dim == 2  # rope_parameters.partial_rotary_factor 0.5 wins over the top-level 0.25
    assert cfg.layer_types == [0, 1]


@pytest.mark.parametrize("mistake", ["no_lora", "plain_norm", "swap_layers"])
def test_golden_catches_planted_mistakes(tiny, mistake):
    cfg, weights, head, golden = tiny
    w = dict(weights)
    c = O.QwenConfig(**{**cfg.__dict__})
    if mistake == "no_lora":
        from safetensors.numpy import load_file
        import pathlib
        w = load_file(str(pathlib.Path(__file__).parent / "golden" / "tiny_kev" / "model.safetensors"))
    elif mistake == "plain_norm":
        for k in list(w):
            if k.endswith("layernorm.weight"):
                w[k] = w[k] - 1.0  # the oracle adds 1: net effect is a plain-weight norm
    elif mistake == "swap_layers":
        c.layer_types = [1, 0]
        for k in list(w):
            if ".layers.0." in k:
                w[k.replace(".layers.0.", ".layers.1.")] = weights[k]
            if ".layers.1." in k:
                w[k.replace(".layers.1.", ".layers.0.")] = weights[k]
    worst_l, worst_p, _ = _golden_errors(c, w, head, golden)
    assert worst_l > 2e-4 or worst_p > 2e-5, (mistake, worst_l, worst_p)


# ---------------------------------------------------------------------------
# gated delta rule
# ---------------------------------------------------------------------------

def _gdn_inputs(seed, T, H, dk, dv):
    q = O.l2norm(O.normal(seed, 1, (T, H, dk))) * np.float32(dk ** -0.5)
    k = O.l2norm(O.normal(seed, 2, (T, H, dk)))
    v = O.normal(seed, 3, (T, H, dv))
    beta = (1.0 / (1.0 + np.exp(-O.normal(seed, 4, (T, H))))).astype(np.float32)
    g = (-np.log1p(np.exp(O.normal(seed, 5, (T, H)))) * 0.5).astype(np.float32)
    return q, k, v, g, beta


def test_delta_rule_split_continuation_is_bit_equal():
    # delta_cpu.rs:221-243: first token then the tail from the carried state == whole
    T, H, dk, dv = 37, 3, 16, 8
    q, k, v, g, beta = _gdn_inputs(11, T, H, dk, dv)
    s0 = O.normal(12, 6, (1, H, dk, dv), std=0.1)
    o_all, s_all = O.gated_delta_rule(q, k, v, g, beta, [0, T], s0)
    for cut in (1, 16, 36):
        o1, s1 = O.gated_delta_rule(q[:cut], k[:cut], v[:cut], g[:cut], beta[:cut], [0, cut], s0)
        o2, s2 = O.gated_delta_rule(q[cut:], k[cut:], v[cut:], g[cut:], beta[cut:], [0, T - cut], s1)
        assert np.array_equal(np.concatenate([o1, o2]).view(np.uint32), o_all.view(np.uint32))
        assert np.array_equal(s2.view(np.uint32), s_all.view(np.uint32))


def test_delta_rule_varlen_equals_per_sequence():
    lens = [5, 64, 1, 30]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q, k, v, g, beta = _gdn_inputs(13, int(cu[-1]), 2, 8, 8)
    o, s = O.gated_delta_rule(q, k, v, g, beta, cu)
    for i in range(len(lens)):
        a, b = cu[i], cu[i + 1]
        oi, si = O.gated_delta_rule(q[a:b], k[a:b], v[a:b], g[a:b], beta[a:b], [0, b - a])
        assert np.array_equal(o[a:b], oi) and np.array_equal(s[i], si[0])


def test_delta_rule_closed_forms():
    H, dk, dv = 2, 8, 4
    q, k, v, g, beta = _gdn_inputs(17, 1, H, dk, dv)
    # one token from a zero state: S = beta k v^T, o = beta (k.q) v
    o, s = O.gated_delta_rule(q, k, v, g, beta, [0, 1])
    for h in range(H):
        expect_s = beta[0, h] * np.outer(k[0, h], v[0, h])
        np.testing.assert_allclose(s[0, h], expect_s, rtol=1e-6, atol=1e-7)
        np.testing.assert_allclose(o[0, h], beta[0, h] * float(k[0, h] @ q[0, h]) * v[0, h], rtol=1e-5,
                                   atol=1e-7)
    # g = 0 and beta = 0: the state never changes and o_t = S0^T q_t
    T = 9
    q, k, v, g, beta = _gdn_inputs(19, T, H, dk, dv)
    s0 = O.normal(20, 7, (1, H, dk, dv))
    o, s = O.gated_delta_rule(q, k, v, np.zeros_like(g), np.zeros_like(beta), [0, T], s0)
    assert np.array_equal(s, s0)
    for t in range(T):
        for h in range(H):
            np.testing.assert_allclose(o[t, h], s0[0, h].T @ q[t, h], rtol=1e-5, atol=1e-6)
    # beta = 1 with a unit key writes v exactly along k: S^T k == v after the update
    kk = np.zeros((1, 1, dk), np.float32)
    kk[0, 0, 3] = 1.0
    vv = O.normal(21, 8, (1, 1, dv))
    _, s = O.gated_delta_rule(kk, kk, vv, np.zeros((1, 1), np.float32), np.ones((1, 1), np.float32), [0, 1],
                              O.normal(22, 9, (1, 1, dk, dv)))
    np.testing.assert_allclose(s[0, 0].T @ kk[0, 0], vv[0, 0], rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# paged KV and attention
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("page_size", [16, 32, 64, 128, 256])
def test_paged_write_page_order_bitwise(page_size):
    # kv_pages.rs:583-630: materialize == concatenation in token order, for each P
    lens = [1, page_size - 1, page_size, 3 * page_size + 5]
    hkv, d = 2, 8
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n = int(cu[-1])
    max_pages = max((L + page_size - 1) // page_size for L in lens)
    num_pages = sum((L + page_size - 1) // page_size for L in lens) + 3
    perm = O.permutation(5, 0, num_pages)
    bt = np.full((len(lens), max_pages), -1, np.int32)
    p = 0
    for s, L in enumerate(lens):
        for j in range((L + page_size - 1) // page_size):
            bt[s, j] = perm[p]
            p += 1
    k = O.bf16_bits(O.normal(1, 0, (n, hkv, d)))
    v = O.bf16_bits(O.normal(1, 1, (n, hkv, d)))
    kp = np.full((num_pages, hkv, page_size, d), 0xFFFF, np.uint16)
    vp = kp.copy()
    pos = np.concatenate([np.arange(L) for L in lens]).astype(np.int32)
    O.paged_kv_write(k, v, cu, pos, bt, page_size, kp, vp)
    for s, L in enumerate(lens):
        pages = [kp[bt[s, j]] for j in range((L + page_size - 1) // page_size)]
        mat = np.concatenate(pages, axis=1)[:, :L]  # [Hkv, L, d]
        assert np.array_equal(mat.transpose(1, 0, 2), k[cu[s]:cu[s + 1]])
    used = set(bt[bt >= 0].tolist())
    for pg in range(num_pages):
        if pg not in used:
            assert (kp[pg] == 0xFFFF).all()


def _dense_pools(k, v, T):
    """One page of T rows holding [Hkv, T, d]: the reference's materialized K/V."""
    return (np.ascontiguousarray(k.transpose(1, 0, 2))[None], np.ascontiguousarray(v.transpose(1, 0, 2))[None])


@pytest.mark.parametrize("page_size", [16, 64])
def test_paged_attention_equals_dense(page_size):
    T, hq, hkv, d = 70, 4, 2, 16
    q = O.normal(3, 0, (T, hq, d))
    k = O.normal(3, 1, (T, hkv, d))
    v = O.normal(3, 2, (T, hkv, d))
    scale = 1.0 / math.sqrt(d)
    kd, vd = _dense_pools(k, v, T)
    dense = O.paged_attention(q, kd, vd, [[0]], [0, T], [T], T, scale)
    npages = (T + page_size - 1) // page_size
    perm = O.permutation(9, 0, npages + 4)[:npages]
    kp = np.zeros((npages + 4, hkv, page_size, d), np.float32)
    vp = np.zeros_like(kp)
    O.paged_kv_write(k, v, [0, T], np.arange(T), perm[None, :], page_size, kp, vp)
    paged = O.paged_attention(q, kp, vp, perm[None, :], [0, T], [T], page_size, scale)
    np.testing.assert_allclose(paged, dense, rtol=0, atol=0)
    # brute force in float64 on the dense layout (GQA: head h reads kv head h // 2)
    for h in range(hq):
        kh, vh = k[:, h // 2].astype(np.float64), v[:, h // 2].astype(np.float64)
        s = (q[:, h].astype(np.float64) @ kh.T) * scale
        s[np.triu_indices(T, 1)] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        np.testing.assert_allclose(dense[:, h], p @ vh, rtol=1e-5, atol=1e-5)


def test_attention_future_poisoning_and_first_row():
    # kv_pages.rs: changing a future value changes only later queries; row 0 returns v_0
    T, hq, hkv, d = 40, 2, 1, 8
    q = O.normal(4, 0, (T, hq, d))
    k = O.normal(4, 1, (T, hkv, d))
    v = O.normal(4, 2, (T, hkv, d))
    kd, vd = _dense_pools(k, v, T)
    a = O.paged_attention(q, kd, vd, [[0]], [0, T], [T], T, 0.3)
    v2 = v.copy()
    v2[25] += 100.0
    kd2, vd2 = _dense_pools(k, v2, T)
    b = O.paged_attention(q, kd2, vd2, [[0]], [0, T], [T], T, 0.3)
    assert np.array_equal(a[:25], b[:25]) and not np.allclose(a[25:], b[25:])
    assert np.array_equal(a[0, 0], v[0, 0]) and np.array_equal(a[0, 1], v[0, 0])


def test_attention_prefix_offset_matches_whole():
    # a suffix of queries with context_lens = prefix + suffix == the same rows of the whole
    T, hq, hkv, d, P = 50, 2, 1, 8, 16
    q = O.normal(6, 0, (T, hq, d))
    k = O.normal(6, 1, (T, hkv, d))
    v = O.normal(6, 2, (T, hkv, d))
    npg = (T + P - 1) // P
    kp = np.zeros((npg, hkv, P, d), np.float32)
    vp = np.zeros_like(kp)
    bt = np.arange(npg, dtype=np.int32)[None]
    O.paged_kv_write(k, v, [0, T], np.arange(T), bt, P, kp, vp)
    whole = O.paged_attention(q, kp, vp, bt, [0, T], [T], P, 0.25)
    tail = O.paged_attention(q[20:], kp, vp, bt, [0, T - 20], [T], P, 0.25)
    assert np.array_equal(whole[20:], tail)


# ---------------------------------------------------------------------------
# conv, norms, rope, calibration
# ---------------------------------------------------------------------------

def test_conv_tap_order_and_continuation():
    T, Cc, K = 12, 5, 4
    w = O.normal(8, 0, (Cc, K))
    impulse = np.zeros((T, Cc), np.float32)
    impulse[0] = 1.0
    out, _ = O.causal_conv1d_silu(impulse, w)
    # an impulse at t=0 reaches output t through tap K-1-t: out[t] = silu(w[:, K-1-t])
    for t in range(K):
        expect = w[:, K - 1 - t] / (1 + np.exp(-w[:, K - 1 - t]))
        np.testing.assert_allclose(out[t], expect, rtol=1e-6)
    assert np.all(out[K:] == 0)
    x = O.normal(8, 1, (T, Cc))
    whole, _ = O.causal_conv1d_silu(x, w)
    first, tail = O.causal_conv1d_silu(x[:7], w, want_tail=True)
    second, _ = O.causal_conv1d_silu(x[7:], w, history=tail)
    assert np.array_equal(np.concatenate([first, second]), whole)
    assert np.array_equal(tail, x[4:7].T)


def test_norms_closed_forms():
    x = O.normal(2, 0, (3, 16))
    w = O.normal(2, 1, (16,))
    y = O.rms_norm_effective(x, w, 1e-6)
    for r in range(3):
        rms = math.sqrt(float((x[r].astype(np.float64) ** 2).mean()) + 1e-6)
        np.testing.assert_allclose(y[r], x[r] / rms * w, rtol=1e-5)
    n = O.l2norm(x)
    np.testing.assert_allclose((n.astype(np.float64) ** 2).sum(1), 1.0, rtol=1e-5)
    z = np.zeros_like(x)  # silu(0) = 0 kills the gated norm
    assert np.all(O.rms_norm_gated(x, z, w, 1e-6) == 0)


def test_rope_rotation_invariants():
    rd, d, theta = 8, 12, 1e7
    pos = np.arange(40, dtype=np.int32)
    c, s = O.rope_cos_sin(rd, theta, pos)
    x = O.normal(3, 0, (40, 1, d))
    y = O.apply_rope(x, rd, c, s)
    # position 0 is the identity; rotation keeps each (i, i+rd/2) pair's norm; the pass dims are untouched
    assert np.array_equal(y[0], x[0])
    half = rd // 2
    for i in range(half):
        np.testing.assert_allclose(np.hypot(y[:, 0, i], y[:, 0, i + half]),
                                   np.hypot(x[:, 0, i], x[:, 0, i + half]), rtol=1e-5)
    assert np.array_equal(y[:, :, rd:], x[:, :, rd:])
    # relative position: q(m).k(n) depends on m - n only
    q = np.repeat(O.normal(3, 1, (1, 1, d)), 40, 0)
    k = np.repeat(O.normal(3, 2, (1, 1, d)), 40, 0)
    qr, kr = O.apply_rope(q, rd, c, s), O.apply_rope(k, rd, c, s)
    dots = [float(qr[m, 0, :rd] @ kr[m - 5, 0, :rd]) for m in range(5, 40)]
    np.testing.assert_allclose(dots, dots[0], rtol=2e-4, atol=2e-4)
    # pair 0 turns by exactly pos radians (inv_freq_0 = theta^0 = 1)
    np.testing.assert_allclose(c[:, 0], np.cos(pos.astype(np.float32)), rtol=1e-6, atol=1e-6)


def test_rope_frequency_ladder_special_values():
    """The frequency ladder of the rotary table (qwen3_5.rs:226-232) at points fixed by the
    textbook RoPE: the pair halfway up the ladder turns by theta^-1/2 per position, the pairs
    are geometric with ratio theta^-2/rd, and the halves of each row repeat (cat(freqs, freqs))."""
    for theta, rd in ((1e4, 8), (1e7, 128), (1.6e5, 64)):
        c, s = O.rope_cos_sin(rd, theta, np.array([1], np.int32))
        ang = np.arctan2(s[0].astype(np.float64), c[0].astype(np.float64))
        half = rd // 2
        np.testing.assert_allclose(ang[:half], ang[half:], rtol=0, atol=0)
        np.testing.assert_allclose(ang[rd // 4], theta ** -0.5, rtol=2e-6)
        np.testing.assert_allclose(ang[1:half] / ang[:half - 1], theta ** (-2.0 / rd), rtol=2e-6)


def test_calibrate_semantics():
    p = O.calibrate([1.0, 2.0, 3.0], 1.3)
    e = np.exp((np.array([1.0, 2.0, 3.0]) - 3.0) / 1.3)
    np.testing.assert_allclose(p, e / e.sum(), rtol=1e-6)
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-6
    for bad in ([1.0, float("nan")], [float("inf"), 0.0]):
        with pytest.raises(ValueError):
            O.calibrate(bad, 1.0)
    with pytest.raises(ValueError):
        O.calibrate([1.0], 0.0)


def test_rng_streams():
    a = O.normal(42, 0, (10001,))
    assert np.array_equal(a, O.normal(42, 0, (10001,)))
    assert not np.array_equal(a, O.normal(42, 1, (10001,)))
    big = O.normal(1, 0, (200000,))
    assert abs(float(big.mean())) < 0.01 and abs(float(big.std()) - 1) < 0.01
    perm = O.permutation(3, 0, 4096)
    assert sorted(perm.tolist()) == list(range(4096))
    ints = O.uniform_int(3, 1, 1000, 64, 2048)
    assert ints.min() >= 64 and ints.max() <= 2048
    assert O.bf16_bits(np.float32([1.0, -2.5, 3.14159274]))[0] == 0x3F80
    assert O.round_bf16(np.float32([1.00390625]))[0] == np.float32(1.0)  # tie rounds to even


# ---------------------------------------------------------------------------
# ModernBERT (Laya backend)
# ---------------------------------------------------------------------------

def synth4_bert_weights():
    """The seeded 4-layer ModernBERT of tests/golden/modernbert/cases.json (`model.*` names)."""
    H, L, I, V = 64, 4, 96, 1000
    shapes = {"embeddings.tok_embeddings.weight": (V, H), "embeddings.norm.weight": (H,), "final_norm.weight": (H,)}
    for l in range(L):
        p = f"layers.{l}."
        shapes.update({p + "attn_norm.weight": (H,), p + "attn.Wqkv.weight": (3 * H, H), p + "attn.Wo.weight": (H, H),
                       p + "mlp_norm.weight": (H,), p + "mlp.Wi.weight": (2 * I, H), p + "mlp.Wo.weight": (H, I)})
    w = {}
    for idx, name in enumerate(sorted(shapes)):
        if name.endswith("norm.weight"):
            mean, std = 1.0, 0.05
        else:
            mean, std = 0.0, {"mlp.Wi.weight": 0.5, "mlp.Wo.weight": 0.2}.get(name.split(".", 2)[-1], 0.05)
        w["model." + name] = O.normal(20261201, 700 + idx, shapes[name], mean, std)
    cfg = O.BertConfig(hidden_size=H, num_hidden_layers=L, num_attention_heads=4, intermediate_size=I, vocab_size=V,
                       global_attn_every_n_layers=3, local_attention=16, global_rope_theta=160000.0,
                       local_rope_theta=10000.0)
    return cfg, w


BERT_TOL = 2e-5  # fp32 oracle vs the golden vectors, absolute on unit-scale LayerNorm outputs


@pytest.fixture(scope="module")
def bert_vectors(golden_dir):
    from safetensors.numpy import load_file

    return load_file(str(golden_dir / "modernbert" / "vectors.safetensors"))


def test_modernbert_oracle_matches_public_definition(golden_dir, bert_vectors):
    """The oracle's ModernBERT forward against golden vectors from an independent
    implementation of the public definition (tests/golden/make_modernbert_vectors.py): the
    reference's tiny_modernbert checkpoint, and a seeded 4-layer model with global and
    local (window 16) layers and distinct RoPE thetas; fp32, 2e-5 absolute on unit-scale
    LayerNorm outputs."""
    cfg, w = O.load_tiny_modernbert(golden_dir / "tiny_modernbert")
    rows = [bert_vectors[f"tiny.ids{i}"].tolist() for i in range(2)]
    for got, exp in zip(O.BertModel(cfg, w).forward(rows), (bert_vectors["tiny.hidden0"], bert_vectors["tiny.hidden1"])):
        assert float(np.abs(got - exp).max()) < BERT_TOL
    cfg, w = synth4_bert_weights()
    rows = [bert_vectors[f"synth4.ids{i}"].tolist() for i in range(2)]
    outs = O.BertModel(cfg, w).forward(rows)
    for got, exp in zip(outs, (bert_vectors["synth4.hidden0"], bert_vectors["synth4.hidden1"])):
        assert float(np.abs(got - exp).max()) < BERT_TOL


@pytest.mark.parametrize("mistake", ["window_off_by_one", "tanh_gelu", "swapped_thetas", "no_attn_norm"])
def test_modernbert_vectors_catch_planted_mistakes(bert_vectors, mistake):
    """Each plausible mistake moves the seeded 4-layer model's output at least 10x past the
    parity tolerance, so the golden vectors pin these details."""
    import dataclasses

    cfg, w = synth4_bert_weights()
    rows = [bert_vectors[f"synth4.ids{i}"].tolist() for i in range(2)]
    if mistake == "window_off_by_one":
        cfg = dataclasses.replace(cfg, local_attention=14)
    elif mistake == "swapped_thetas":
        cfg = dataclasses.replace(cfg, global_rope_theta=10000.0, local_rope_theta=160000.0)
    elif mistake == "no_attn_norm":
        w = {k: v for k, v in w.items() if k != "model.layers.0.attn_norm.weight"}
    m = O.BertModel(cfg, w)
    if mistake == "tanh_gelu":  # the tanh approximation in place of the exact erf form
        outs = _bert_forward_numpy(cfg, w, rows, lambda x: 0.5 * x * (1 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3))))
    else:
        outs = m.forward(rows)
    err = max(float(np.abs(g - bert_vectors[f"synth4.hidden{i}"]).max()) for i, g in enumerate(outs))
    assert err > 10 * BERT_TOL, (mistake, err)


def _bert_forward_numpy(cfg, w, rows, act):
    """A numpy restatement with a pluggable activation (used only to plant a mistake)."""
    H, nh, d, I = cfg.hidden_size, cfg.num_attention_heads, cfg.head_dim, cfg.intermediate_size
    outs = []
    for r in rows:
        T = len(r)
        pos = np.arange(T, dtype=np.int32)
        h = O.layer_norm(w["model.embeddings.tok_embeddings.weight"][r], w["model.embeddings.norm.weight"])
        for l in range(cfg.num_hidden_layers):
            glob = l % cfg.global_attn_every_n_layers == 0
            p = f"model.layers.{l}."
            x = O.layer_norm(h, w[p + "attn_norm.weight"]) if p + "attn_norm.weight" in w else h
            qkv = O.linear(x, w[p + "attn.Wqkv.weight"]).reshape(T, 3, nh, d)
            q, k, v = (np.ascontiguousarray(qkv[:, i]) for i in range(3))
            c, s = O.rope_cos_sin(d, cfg.global_rope_theta if glob else cfg.local_rope_theta, pos)
            q, k = O.apply_rope(q, d, c, s), O.apply_rope(k, d, c, s)
            a = O.bidir_attention(q, k, v, [0, T], -1 if glob else cfg.local_attention // 2)
            h = h + O.linear(a.reshape(T, H), w[p + "attn.Wo.weight"])
            gi = O.linear(O.layer_norm(h, w[p + "mlp_norm.weight"]), w[p + "mlp.Wi.weight"])
            h = h + O.linear((act(gi[:, :I]) * gi[:, I:]).astype(np.float32), w[p + "mlp.Wo.weight"])
        outs.append(O.layer_norm(h, w["model.final_norm.weight"]))
    return outs
