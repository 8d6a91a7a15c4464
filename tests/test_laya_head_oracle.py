"""The oracle's typed Laya head (oracle.laya_head) pinned against PyTorch's own modules.

The reference builds each head layer as `nn.TransformerEncoderLayer` (norm_first, batch_first,
ReLU FFN; crates/huncho-backend/src/candle.rs:502-585) and the scorer as LayerNorm -> Linear ->
GELU(erf) -> Linear (590-694). torch.nn has exactly those modules, so the fp32 oracle must
equal them on the reference's own deterministic test head (tests/support/laya.rs:5-52, restated
by oracle.laya_test_head) and its test input (h[i] = ((17 i mod 239) - 119) / 128, 33 tokens,
d 128, 2 layers: candle.rs:722-757). Planted mistakes (a post-norm layer, GELU in the FFN, no
type embedding) must each move the scores far beyond the tolerance. The selected-last-layer
shortcut of the reference (forward_queries) is an optimisation with equal results and is not
restated.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O

D, LAYERS = 128, 2


def reference_input():
    return np.array([((i * 17 % 239) - 119) / 128 for i in range(33 * D)], np.float32).reshape(33, D)


def torch_head(h, w, qtype, positions, norm_first=True, activation="relu", type_emb=True):
    torch.manual_seed(0)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32))
    z = t(h)[None]
    if type_emb:
        z = z + t(w["type_emb.weight"][qtype])[None, None]
    i = 0
    with torch.no_grad():
        while f"head.layers.{i}.self_attn.in_proj_weight" in w:
            p = f"head.layers.{i}."
            ffn = w[p + "linear1.weight"].shape[0]
            layer = torch.nn.TransformerEncoderLayer(D, max(D // 64, 1), dim_feedforward=ffn, dropout=0.0,
                                                     activation=activation, layer_norm_eps=1e-5, batch_first=True,
                                                     norm_first=norm_first)
            layer.self_attn.in_proj_weight.copy_(t(w[p + "self_attn.in_proj_weight"]))
            layer.self_attn.in_proj_bias.copy_(t(w[p + "self_attn.in_proj_bias"]))
            layer.self_attn.out_proj.weight.copy_(t(w[p + "self_attn.out_proj.weight"]))
            layer.self_attn.out_proj.bias.copy_(t(w[p + "self_attn.out_proj.bias"]))
            for n in ("norm1", "norm2"):
                getattr(layer, n).weight.copy_(t(w[p + n + ".weight"]))
                getattr(layer, n).bias.copy_(t(w[p + n + ".bias"]))
            for n in ("linear1", "linear2"):
                getattr(layer, n).weight.copy_(t(w[p + n + ".weight"]))
                getattr(layer, n).bias.copy_(t(w[p + n + ".bias"]))
            layer.eval()
            z = layer(z)
            i += 1
        m = z[0, torch.as_tensor(positions)]
        y = torch.nn.functional.layer_norm(m, (D,), t(w["scorer.0.weight"]), t(w["scorer.0.bias"]), 1e-5)
        y = torch.nn.functional.linear(y, t(w["scorer.1.weight"]), t(w["scorer.1.bias"]))
        y = torch.nn.functional.gelu(y, approximate="none")
        y = torch.nn.functional.linear(y, t(w["scorer.3.weight"]), t(w["scorer.3.bias"]))
    return y[:, 0].numpy()


@pytest.fixture(scope="module")
def head():
    return O.laya_test_head(D, LAYERS)


@pytest.mark.parametrize("qtype", [0, 1, 2])
@pytest.mark.parametrize("positions", [[32, 0, 9, 0], list(range(32, -1, -1))])
def test_oracle_head_equals_torch_modules(head, qtype, positions):
    h = reference_input()
    ours = O.laya_head(h, head, qtype, positions)
    ref = torch_head(h, head, qtype, positions)
    err = float(np.abs(ours - ref).max() / max(np.abs(ref).max(), 1e-30))
    assert err < 1e-5, err


@pytest.mark.parametrize("mistake", ["post_norm", "gelu_ffn", "no_type_emb"])
def test_planted_mistakes_are_visible(head, mistake):
    h = reference_input()
    pos = list(range(33))
    ref = O.laya_head(h, head, 1, pos)
    kw = {"post_norm": dict(norm_first=False), "gelu_ffn": dict(activation="gelu"),
          "no_type_emb": dict(type_emb=False)}[mistake]
    wrong = torch_head(h, head, 1, pos, **kw)
    err = float(np.abs(ref - wrong).max() / max(np.abs(ref).max(), 1e-30))
    assert err > 1e-3, (mistake, err)


def test_bf16_flow_stays_close(head):
    """The bf16 flow (every op rounded) stays within bf16 distance of fp32 on this head."""
    h = reference_input()
    a = O.laya_head(h, head, 2, [32, 0, 9])
    b = O.laya_head(h, head, 2, [32, 0, 9], bf16=True)
    assert float(np.abs(a - b).max() / np.abs(a).max()) < 5e-2
