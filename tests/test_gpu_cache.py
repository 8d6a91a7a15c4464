"""The device prefix cache (hk_kev_cache) against fresh forwards and the oracle.

Properties the reference's chunked-prefill and prefix-cache tests hold (crates/huncho-backend/
tests/chunked_prefill.rs, prefix_cache.rs: continued == whole; forks never see each other;
a parent is unchanged by its branches, kv_pages.rs:307-341 copy-on-write tails):
  * prefill(prefix) + continuation(suffix) == a fresh forward of prefix + suffix, for split
    points on and off page (16) and chunk (64) boundaries, and for several rows at once;
  * forks of one parent with different suffixes == their fresh forwards, and the parent,
    continued afterwards, == its own fresh forward (the shared partial tail page was copied);
  * fork_batch leaves the parent and the pool as they were; released handles free their pages;
  * failures (unknown handle, empty row, context overflow, exhausted pool) commit nothing.
fp16 activations: calibrated probabilities within 1e-3 of the fp32 oracle's full-sequence
forward (the qualification gate, conformance.rs:20-48), and continued vs fresh on the GPU
within 2e-3 (different chunk partitions of the same recurrence round differently in fp16).
fp32 activations: continued and forked rows within 2e-5 of the oracle and of a fresh forward.
(The bf16 cache at the Kev shape itself is in test_gpu_workloads.py.)
"""
import numpy as np
import pytest
import torch

from huncho_amd import abi
from huncho_amd.kev import KevCache, KevModel, KevShape, synthetic_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SEED = 777
TEMP = 1.3
SHAPE = dict(hidden=256, n_layers=4, n_heads=2, n_kv_heads=1, intermediate=512, vocab=1000, lin_n_k_heads=2,
             lin_n_v_heads=2, rotary_dim=64, rope_theta=10000.0, n_out=5, max_context=1024)


@pytest.fixture(scope="module")
def setup():
    from huncho_amd.ops import context_for_torch

    ctx = context_for_torch(0)
    shape = KevShape(**SHAPE)
    weights = synthetic_weights(shape, SEED, std=0.05)
    model = KevModel(ctx, shape, weights, torch.float16)
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
    head_w = f["decision_head.weight"]

    def oracle_probs(tokens):
        h = ref.forward(np.asarray(tokens, np.int64))
        return O.calibrate((h[-1] @ head_w.T).astype(np.float32), TEMP)

    yield dict(ctx=ctx, model=model, oracle_probs=oracle_probs)
    model.close()
    ctx.close()


def toks(stream, n):
    return abi.synth_uniform_int(SEED, stream, n, 0, SHAPE["vocab"] - 1).tolist()


def fresh_probs(model, rows):
    return model.forward_batch(rows, temperature=TEMP)[1]


@pytest.mark.parametrize("split", [1, 17, 64, 100])
def test_continuation_equals_whole(setup, split):
    model, cache = setup["model"], KevCache(setup["model"], max_pages=64)
    full = toks(10 + split, 150)
    h = cache.prefill(full[:split])
    assert cache.tokens(h) == split
    _, p_cont, _ = cache.continue_rows([h], [full[split:]], TEMP)
    assert cache.tokens(h) == len(full)
    p_fresh = fresh_probs(model, [full])
    p_ref = setup["oracle_probs"](full)
    d_fresh, d_ref = float(np.abs(p_cont - p_fresh).max()), float(np.abs(p_cont[0] - p_ref).max())
    print(f"split {split}: continued vs fresh {d_fresh:.2e}, vs fp32 oracle {d_ref:.2e}")
    assert d_fresh < 2e-3 and d_ref < 1e-3, (d_fresh, d_ref)
    cache.release(h)
    assert cache.stats() == (0, 64)
    cache.close()


def test_rows_continue_together_and_chain(setup):
    """Three handles with different cached lengths continue in one call; one of them then
    continues again (three segments)."""
    model, cache = setup["model"], KevCache(setup["model"], max_pages=64)
    seqs = [toks(30 + i, L) for i, L in enumerate([90, 40, 161])]
    cuts = [33, 16, 100]
    hs = [cache.prefill(s[:c]) for s, c in zip(seqs, cuts)]
    _, p_cont, _ = cache.continue_rows(hs, [s[c:] for s, c in zip(seqs, cuts)], TEMP)
    p_fresh = fresh_probs(model, seqs)
    assert float(np.abs(p_cont - p_fresh).max()) < 2e-3
    more = toks(40, 29)
    _, p3, _ = cache.continue_rows([hs[1]], [more], TEMP)
    whole = seqs[1] + more
    d = float(np.abs(p3[0] - setup["oracle_probs"](whole)).max())
    assert d < 1e-3, d
    assert cache.tokens(hs[1]) == len(whole)
    for h in hs:
        cache.release(h)
    cache.close()


def test_forks_are_private_and_parent_unchanged(setup):
    """Prefix of 21 tokens: its second page is partial and shared by the parent and both forks."""
    model, cache = setup["model"], KevCache(setup["model"], max_pages=64)
    prefix = toks(50, 21)
    s1, s2, s3 = toks(51, 30), toks(52, 7), toks(53, 44)
    parent = cache.prefill(prefix)
    live, free_after_prefill = cache.stats()
    c1, c2 = cache.fork(parent), cache.fork(parent)
    assert cache.stats() == (3, free_after_prefill)  # forks share the parent's pages
    _, p_forks, _ = cache.continue_rows([c1, c2], [s1, s2], TEMP)
    p_fresh = fresh_probs(model, [prefix + s1, prefix + s2])
    assert float(np.abs(p_forks - p_fresh).max()) < 2e-3
    # the parent continues after its branches appended to copies of the shared tail page
    _, p_parent, _ = cache.continue_rows([parent], [s3], TEMP)
    d = float(np.abs(p_parent[0] - setup["oracle_probs"](prefix + s3)).max())
    print(f"parent after forks vs fp32 oracle: {d:.2e}")
    assert d < 1e-3, d
    # a fork taken now sees the parent's tokens, not a branch's
    c3 = cache.fork(parent)
    assert cache.tokens(c3) == len(prefix) + len(s3)
    for h in (c1, c2, c3, parent):
        cache.release(h)
    assert cache.stats() == (0, 64)
    cache.close()


def test_parent_and_fork_continue_together(setup):
    """A parent and its fork share a partial tail page (21-token prefix) and continue in one
    call: each gets a private copy of the tail, the shared page is returned to the pool (no
    page is lost), and both equal their fresh forwards."""
    model, cache = setup["model"], KevCache(setup["model"], max_pages=64)
    prefix = toks(55, 21)
    s1, s2 = toks(56, 9), toks(57, 30)
    parent = cache.prefill(prefix)
    child = cache.fork(parent)
    _, p, _ = cache.continue_rows([parent, child], [s1, s2], TEMP)
    p_fresh = fresh_probs(model, [prefix + s1, prefix + s2])
    assert float(np.abs(p - p_fresh).max()) < 2e-3
    # pages held now: the shared full first page, a private copy of the tail for each, and the
    # child's 2 new pages (parent 30 tokens, child 51)
    assert cache.stats() == (2, 64 - 5)
    cache.release(parent)
    cache.release(child)
    assert cache.stats() == (0, 64)
    cache.close()


def test_fork_batch_leaves_parent_and_pool(setup):
    model, cache = setup["model"], KevCache(setup["model"], max_pages=64)
    prefix = toks(60, 48)  # three full pages: branches append to fresh pages only
    parent = cache.prefill(prefix)
    before = cache.stats()
    suffixes = [toks(61 + i, L) for i, L in enumerate([5, 12, 12, 30])]
    _, probs = cache.fork_batch(parent, suffixes, TEMP)
    p_fresh = fresh_probs(model, [prefix + s for s in suffixes])
    assert float(np.abs(probs - p_fresh).max()) < 2e-3
    assert cache.stats() == before and cache.tokens(parent) == len(prefix)
    cache.release(parent)
    cache.close()


def test_failures_commit_nothing(setup):
    cache = KevCache(setup["model"], max_pages=4, max_handles=3)  # 4 pages of 16 tokens
    h = cache.prefill(toks(70, 20))
    with pytest.raises(abi.HkError):
        cache.continue_rows([h + 1000], [[1, 2]])
    with pytest.raises(abi.HkError):
        cache.continue_rows([h], [[]])
    with pytest.raises(abi.HkError):  # 20 + 50 tokens need 5 pages of the 4
        cache.continue_rows([h], [toks(71, 50)])
    assert cache.tokens(h) == 20 and cache.stats() == (1, 2)
    with pytest.raises(abi.HkError):  # the same handle twice in one call
        cache.continue_rows([h, h], [[1], [2]])
    with pytest.raises(abi.HkError):  # beyond max_context (1024)
        cache.continue_rows([h], [[1] * 1010])
    a, b = cache.fork(h), cache.fork(h)
    with pytest.raises(abi.HkError):  # max_handles = 3
        cache.open()
    for x in (a, b, h):
        cache.release(x)
    with pytest.raises(abi.HkError):
        cache.release(h)
    assert cache.stats() == (0, 4)
    cache.close()


# ---------------------------------------------------------------------------
# fp32 activations: the unfused Gated DeltaNet path (gdn_prep + gdn_chunk_f32) with the
# cache's per-sequence state and conv-tail rows
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def model32(setup):
    shape = KevShape(**SHAPE)
    m = KevModel(setup["ctx"], shape, synthetic_weights(shape, SEED, std=0.05), torch.float32)
    yield m
    m.close()


def test_fp32_continuation_and_fork(setup, model32):
    """fp32: prefill + continuation at splits on and off page/chunk boundaries, and a parent
    with a fork continuing together from a shared partial tail page, each within the fp32
    probability gate (2e-5, crates/huncho-backend/tests/kev_reference.rs:79) of the oracle's
    full-sequence forward and of a fresh fp32 forward."""
    cache = KevCache(model32, max_pages=64)
    full = toks(80, 150)
    hs = [cache.prefill(full[:cut]) for cut in (17, 64, 100)]
    _, p_cont, _ = cache.continue_rows(hs, [full[cut:] for cut in (17, 64, 100)], TEMP)
    p_ref = setup["oracle_probs"](full)
    p_fresh = fresh_probs(model32, [full])[0]
    d_ref, d_fresh = float(np.abs(p_cont - p_ref).max()), float(np.abs(p_cont - p_fresh).max())
    print(f"fp32 continuation: vs fp32 oracle {d_ref:.2e}, vs fresh {d_fresh:.2e}")
    assert d_ref < 2e-5 and d_fresh < 2e-5, (d_ref, d_fresh)
    for h in hs:
        cache.release(h)
    prefix, s1, s2 = toks(81, 21), toks(82, 9), toks(83, 40)
    parent = cache.prefill(prefix)
    child = cache.fork(parent)
    _, p, _ = cache.continue_rows([parent, child], [s1, s2], TEMP)
    for row, whole in zip(p, (prefix + s1, prefix + s2)):
        d = float(np.abs(row - setup["oracle_probs"](whole)).max())
        assert d < 2e-5, d
    cache.release(parent)
    cache.release(child)
    assert cache.stats() == (0, 64)
    cache.close()


# ---------------------------------------------------------------------------
# exact-prefix retention (prefill_cached) and resumable chunked prefill
# ---------------------------------------------------------------------------

def retention_bytes(n_tokens, esz=2):
    """ModelCache::retention_bytes (qwen3_5.rs:1161-1185) on the cache's storage."""
    shape = KevShape(**SHAPE)
    n_attn = sum(1 for t in shape.layer_types if t == 1)
    n_gdn = shape.n_layers - n_attn
    page_bytes = shape.n_kv_heads * shape.page_size * shape.head_dim * esz
    pages = -(-n_tokens // shape.page_size)
    state = shape.lin_n_v_heads * 128 * 128 * 4
    conv = shape.conv_dim * 3 * esz
    return 8 * n_tokens + 512 + shape.n_layers * 512 + n_attn * pages * 2 * page_bytes + n_gdn * (state + conv)


def test_prefill_cached_hit_clones_the_prefix(setup):
    """A retained prefix is cloned on an identical request (hit, no model work); the clone and the
    original continue identically, and continuing them leaves the snapshot unchanged."""
    model, cache = setup["model"], KevCache(setup["model"], max_pages=64)
    prefix, s1, s2 = toks(90, 100), toks(91, 20), toks(92, 33)
    budget = 1 << 40
    w = abi.PrefillWork()
    h1, hit1 = cache.prefill_cached(prefix, budget, work=w)
    assert not hit1 and (w.forward_calls, w.processed_tokens, w.chunked_prefills) == (1, 100, 0)
    assert cache.prefix_stats() == (1, retention_bytes(100))
    h2, hit2 = cache.prefill_cached(prefix, budget, work=w)
    assert hit2 and (w.forward_calls, w.processed_tokens) == (1, 100) and cache.tokens(h2) == 100
    _, p1, _ = cache.continue_rows([h1], [s1], TEMP)
    _, p2, _ = cache.continue_rows([h2], [s1], TEMP)
    assert np.array_equal(p1, p2)  # the same pages and state, the same computation
    h3, hit3 = cache.prefill_cached(prefix, budget)
    assert hit3
    _, p3, _ = cache.continue_rows([h3], [s2], TEMP)
    d = float(np.abs(p3[0] - setup["oracle_probs"](prefix + s2)).max())
    print(f"clone of a retained prefix, continued: vs fp32 oracle {d:.2e}")
    assert d < 1e-3, d
    for h in (h1, h2, h3):
        cache.release(h)
    assert cache.stats()[0] == 0 and cache.stats()[1] < 64  # the snapshot still holds its pages
    cache.clear_prefixes()
    assert cache.prefix_stats() == (0, 0) and cache.stats() == (0, 64)
    cache.close()


def test_prefill_cached_chunks_and_budget(setup):
    """Chunked prefill equals the whole-prefix prefill; the byte budget decides what is retained
    and evicts first in, first out."""
    model, cache = setup["model"], KevCache(setup["model"], max_pages=64)
    a, b, suffix = toks(93, 150), toks(94, 40), toks(95, 17)
    w = abi.PrefillWork()
    h, hit = cache.prefill_cached(a, 0, chunk_tokens=64, work=w)  # budget 0: nothing retained
    assert not hit and (w.forward_calls, w.processed_tokens, w.chunked_prefills) == (3, 150, 1)
    assert cache.prefix_stats() == (0, 0)
    _, p, _ = cache.continue_rows([h], [suffix], TEMP)
    d_fresh = float(np.abs(p - fresh_probs(model, [a + suffix])).max())
    d_ref = float(np.abs(p[0] - setup["oracle_probs"](a + suffix)).max())
    print(f"3-chunk prefill + continuation: vs fresh {d_fresh:.2e}, vs fp32 oracle {d_ref:.2e}")
    assert d_fresh < 2e-3 and d_ref < 1e-3, (d_fresh, d_ref)
    cache.release(h)
    # a budget below the prefix's charged bytes retains nothing
    h, _ = cache.prefill_cached(b, retention_bytes(40) - 1)
    assert cache.prefix_stats() == (0, 0)
    cache.release(h)
    # a budget for one: the second prefix evicts the first
    one = max(retention_bytes(40), retention_bytes(150))
    ha, _ = cache.prefill_cached(a, one)
    hb, _ = cache.prefill_cached(b, one)
    assert cache.prefix_stats() == (1, retention_bytes(40))
    ha2, hit_a = cache.prefill_cached(a, one)
    assert not hit_a
    for x in (ha, hb, ha2):
        cache.release(x)
    cache.clear_prefixes()
    assert cache.stats() == (0, 64)
    cache.close()


def test_resumable_prefill(setup):
    """begin / advance_resumable_prefill: one chunk per call, the partial handle can be neither
    forked nor continued, completion retains the prefix, cancelling frees the pages."""
    model, cache = setup["model"], KevCache(setup["model"], max_pages=64)
    prefix, suffix = toks(96, 150), toks(97, 21)
    budget = 1 << 40
    h, hit = cache.begin_resumable(prefix, budget)
    assert not hit and cache.tokens(h) == 0
    with pytest.raises(abi.HkError):
        cache.fork(h)
    with pytest.raises(abi.HkError):
        cache.continue_rows([h], [suffix])
    w = abi.PrefillWork()
    done = [cache.advance_resumable(h, prefix, 64, w) for _ in range(3)]
    assert done == [False, False, True] and cache.tokens(h) == 150
    assert (w.forward_calls, w.processed_tokens, w.chunked_prefills) == (3, 150, 1)
    with pytest.raises(abi.HkError):  # completed: no longer pending
        cache.advance_resumable(h, prefix, 64, w)
    _, p, _ = cache.continue_rows([h], [suffix], TEMP)
    d = float(np.abs(p[0] - setup["oracle_probs"](prefix + suffix)).max())
    print(f"resumable prefill (3 chunks) + continuation: vs fp32 oracle {d:.2e}")
    assert d < 1e-3, d
    h2, hit2 = cache.begin_resumable(prefix, budget)  # retained at completion
    assert hit2 and cache.tokens(h2) == 150
    for x in (h, h2):
        cache.release(x)
    cache.clear_prefixes()
    free0 = cache.stats()[1]
    h3, _ = cache.begin_resumable(toks(98, 100), budget)
    assert not cache.advance_resumable(h3, toks(98, 100), 40)
    cache.release(h3)  # cancel mid-way
    assert cache.stats() == (0, free0) and cache.prefix_stats() == (0, 0)
    cache.close()
