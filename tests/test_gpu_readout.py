"""The readout at request positions (Qwen3_5Backend::readout, crates/huncho-backend/src/
qwen3_5.rs:3196-3255) and the Kev PointerHead scores (kev.rs:161-165) against the oracle's final
hidden states and its pointer_head.

Gates: fp32 activations: pointer scores within 2e-4 absolute of the oracle's (the fp32 raw-logit
gate of crates/huncho-backend/tests/kev_reference.rs:61-87), their calibrated probabilities within
2e-5, hidden rows within 1e-4 absolute. fp16 cached continuation: scores within 2e-2 and
probabilities within 1e-3 of the oracle's fp32 forward of prefix + suffix.
"""
import numpy as np
import pytest
import torch

from huncho_amd import abi
from huncho_amd.kev import KevCache, KevModel, KevShape, synthetic_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SEED = 9090
TEMP = 2.406050072164233  # the Kev fixture's temperature (tests/golden/tiny_kev/head.json)
SHAPE = dict(hidden=256, n_layers=4, n_heads=2, n_kv_heads=1, intermediate=512, vocab=1000, lin_n_k_heads=2,
             lin_n_v_heads=2, rotary_dim=64, rope_theta=10000.0, n_out=0, max_context=1024)
HEAD_DIM = 64


@pytest.fixture(scope="module")
def setup():
    from huncho_amd.ops import context_for_torch

    ctx = context_for_torch(0)
    shape = KevShape(**SHAPE)
    weights = synthetic_weights(shape, SEED, std=0.05)
    cfg = O.QwenConfig(hidden_size=shape.hidden, num_hidden_layers=shape.n_layers,
                       num_attention_heads=shape.n_heads, num_key_value_heads=shape.n_kv_heads,
                       head_dim=shape.head_dim, intermediate_size=shape.intermediate, vocab_size=shape.vocab,
                       rms_norm_eps=shape.eps, layer_types=shape.layer_types,
                       linear_conv_kernel_dim=shape.conv_k, linear_key_head_dim=shape.lin_key_dim,
                       linear_num_key_heads=shape.lin_n_k_heads, linear_num_value_heads=shape.lin_n_v_heads,
                       linear_value_head_dim=shape.lin_v_dim, rope_theta=shape.rope_theta,
                       partial_rotary_factor=shape.rotary_dim / shape.head_dim)
    f = {k: O.bf16_to_f32(v).reshape(v.shape) for k, v in weights.items()}
    ref = O.QwenModel(cfg, f, bf16=False)
    rng = np.random.default_rng(SEED)
    head = {"q_weight": (rng.standard_normal((HEAD_DIM, shape.hidden)) * 0.06).astype(np.float32),
            "q_bias": (rng.standard_normal(HEAD_DIM) * 0.1).astype(np.float32),
            "k_weight": (rng.standard_normal((HEAD_DIM, shape.hidden)) * 0.06).astype(np.float32),
            "k_bias": (rng.standard_normal(HEAD_DIM) * 0.1).astype(np.float32), "head_dim": HEAD_DIM}
    yield dict(ctx=ctx, shape=shape, weights=weights, ref=ref, head=head)
    ctx.close()


def toks(stream, n):
    return abi.synth_uniform_int(SEED, stream, n, 0, SHAPE["vocab"] - 1).tolist()


def test_pointer_readout_fp32(setup):
    """Three rows of 90, 1 and 140 tokens with option positions on page, chunk and row edges
    (and a row reading none): rows and pointer scores against the oracle."""
    model = KevModel(setup["ctx"], setup["shape"], setup["weights"], torch.float32)
    h = setup["head"]
    model.set_pointer_head(h["q_weight"], h["q_bias"], h["k_weight"], h["k_bias"])
    rows = [toks(10, 90), toks(11, 1), toks(12, 140), toks(13, 20)]
    positions = [[3, 15, 16, 63, 64, 89], [0], [0, 50, 127, 128, 139], []]
    hidden, scores, _ = model.forward_readout(rows, positions, want_hidden=True, want_scores=True)
    k = 0
    worst_h = worst_s = worst_p = 0.0
    for r, pos in zip(rows, positions):
        if not pos:
            continue
        hr = setup["ref"].forward(r)
        ref_s = O.pointer_head(hr, pos, h)
        got = scores[k:k + len(pos)]
        worst_h = max(worst_h, float(np.abs(hidden[k:k + len(pos)] - hr[pos]).max()))
        worst_s = max(worst_s, float(np.abs(got - ref_s).max()))
        worst_p = max(worst_p, float(np.abs(O.calibrate(got, TEMP) - O.calibrate(ref_s, TEMP)).max()))
        k += len(pos)
    model.close()
    print(f"pointer readout fp32: hidden {worst_h:.2e}, scores {worst_s:.2e}, probabilities {worst_p:.2e}")
    assert worst_h < 1e-4 and worst_s < 2e-4 and worst_p < 2e-5, (worst_h, worst_s, worst_p)


def test_readout_rejects_positions_outside_rows(setup):
    model = KevModel(setup["ctx"], setup["shape"], setup["weights"], torch.float32)
    with pytest.raises(abi.HkError):
        model.forward_readout([toks(20, 10)], [[10]])
    with pytest.raises(abi.HkError):  # scores without a pointer head
        model.forward_readout([toks(20, 10)], [[3]], want_hidden=False, want_scores=True)
    model.close()


def test_pointer_readout_cached_fp16(setup):
    """A prefix in the cache, two forks continued with suffixes; positions index the suffixes
    (ForwardInput.positions with fork_from): scores against the oracle's fp32 forward of
    prefix + suffix at prefix_len + position."""
    model = KevModel(setup["ctx"], setup["shape"], setup["weights"], torch.float16)
    h = setup["head"]
    model.set_pointer_head(h["q_weight"], h["q_bias"], h["k_weight"], h["k_bias"])
    cache = KevCache(model, max_pages=64)
    prefix = toks(30, 37)
    parent = cache.prefill(prefix)
    forks = [cache.fork(parent), cache.fork(parent)]
    suffixes = [toks(31, 25), toks(32, 70)]
    positions = [[0, 7, 24], [5, 40, 69]]
    _, scores, _ = cache.continue_rows_readout(forks, suffixes, positions, want_hidden=False, want_scores=True)
    k = 0
    worst_s = worst_p = 0.0
    for sfx, pos in zip(suffixes, positions):
        hr = setup["ref"].forward(prefix + sfx)
        ref_s = O.pointer_head(hr, [len(prefix) + p for p in pos], h)
        got = scores[k:k + len(pos)]
        worst_s = max(worst_s, float(np.abs(got - ref_s).max()))
        worst_p = max(worst_p, float(np.abs(O.calibrate(got, TEMP) - O.calibrate(ref_s, TEMP)).max()))
        k += len(pos)
    for x in forks + [parent]:
        cache.release(x)
    cache.close()
    model.close()
    print(f"pointer readout fp16 cached: scores {worst_s:.2e}, probabilities {worst_p:.2e}")
    assert worst_s < 2e-2 and worst_p < 1e-3, (worst_s, worst_p)
