"""Writes the ModernBERT golden vectors in tests/golden/modernbert/ (run here, once; never on a
GPU host). The reference executes ModernBERT through candle-transformers 0.11, which is not
vendored and holds no golden vectors, so these vectors come from an independent
implementation of the public ModernBERT definition, transformers' ModernBertModel (eager
attention, fp32, CPU), configured as the reference's Laya loader configures candle
(crates/huncho-backend/src/candle.rs:157-231): LayerNorm without bias, eps from
layer_norm_eps, the rope_parameters thetas, local_attention, global_attn_every_n_layers,
exact GELU in the GeGLU MLP, and an attention LayerNorm in every layer whose checkpoint
carries one (the tiny_modernbert fixture's layer 0 does; transformers would otherwise make
layer 0's an identity).

Cases:
  tiny      the reference fixture crates/huncho-backend/tests/fixtures/tiny_modernbert
            (copied next to this script), ids [1..5] (candle_integration.rs:39-40) and a
            13-token row;
  synth4    hidden 64, 4 layers (global 0 and 3, local 1 and 2 with window 16), 4 heads,
            GeGLU 96, vocab 1000, thetas 160000 / 10000; seeded normal weights from the
            oracle's RNG (stream 700 + sorted-name index; N(1, 0.05) norms, N(0, 0.5) Wi,
            N(0, 0.2) MLP Wo, N(0, 0.05) the rest); two rows of 37 and 50 ids.
Output: modernbert/vectors.safetensors (inputs and final hidden states) and cases.json.
"""
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
from oracle import oracle as O  # noqa: E402  (seeded RNG only)


def synth4_init(name):
    """(mean, std) of a synth4 tensor: norms around 1; the MLP scaled up so that its GeGLU
    inputs reach the range where exact and tanh-approximated GELU differ."""
    if name.endswith("norm.weight"):
        return 1.0, 0.05
    if name.endswith("mlp.Wi.weight"):
        return 0.0, 0.5
    if name.endswith("mlp.Wo.weight"):
        return 0.0, 0.2
    return 0.0, 0.05


def build(cfg_kw, weights, has_attn_norm0):
    from transformers import ModernBertConfig, ModernBertModel

    n_layers = cfg_kw["num_hidden_layers"]
    every = cfg_kw["global_attn_every_n_layers"]
    layer_types = ["sliding_attention" if i % every else "full_attention" for i in range(n_layers)]
    kw = dict(cfg_kw)
    if len(set(layer_types)) == 1:
        # transformers' config validation wants both layer types present at construction;
        # build with one of each, then set the real layer list (the RoPE table is per type)
        kw["num_hidden_layers"] = 2
        kw["global_attn_every_n_layers"] = 2
    cfg = ModernBertConfig(hidden_activation="gelu", norm_bias=False, attention_bias=False, mlp_bias=False, **kw)
    cfg.num_hidden_layers = n_layers
    cfg.layer_types = layer_types
    cfg._attn_implementation = "eager"
    model = ModernBertModel(cfg).eval()
    if has_attn_norm0:
        model.layers[0].attn_norm = torch.nn.LayerNorm(cfg.hidden_size, eps=cfg.norm_eps, bias=False)
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in weights.items()}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in m or "inv_freq" in m for m in missing), missing
    return model


def run(model, rows):
    outs = []
    with torch.no_grad():
        for r in rows:
            h = model(input_ids=torch.tensor([r], dtype=torch.long)).last_hidden_state[0]
            outs.append(h.numpy().astype(np.float32))
    return outs


def main():
    from safetensors.numpy import load_file, save_file

    out, cases = {}, {}
    # tiny reference fixture
    root = HERE / "tiny_modernbert"
    raw = load_file(str(root / "model.safetensors"))
    cj = json.loads((root / "config.json").read_text())
    w = {k[len("encoder."):]: v for k, v in raw.items() if k.startswith("encoder.")}
    kw = dict(vocab_size=cj["vocab_size"], hidden_size=cj["hidden_size"], num_hidden_layers=cj["num_hidden_layers"],
              num_attention_heads=cj["num_attention_heads"], intermediate_size=cj["intermediate_size"],
              norm_eps=cj["layer_norm_eps"], global_attn_every_n_layers=cj["global_attn_every_n_layers"],
              local_attention=cj["local_attention"], max_position_embeddings=cj["max_position_embeddings"],
              global_rope_theta=cj["rope_parameters"]["full_attention"]["rope_theta"],
              local_rope_theta=cj["rope_parameters"]["sliding_attention"]["rope_theta"],
              pad_token_id=cj["pad_token_id"])
    rows = [[1, 2, 3, 4, 5], [7, 31, 500, 2, 9999, 12, 1, 1, 32767, 64, 3, 8, 100]]
    hs = run(build(kw, w, "layers.0.attn_norm.weight" in w), rows)
    for i, (r, h) in enumerate(zip(rows, hs)):
        out[f"tiny.ids{i}"] = np.asarray(r, np.int32)
        out[f"tiny.hidden{i}"] = h
    cases["tiny"] = {"rows": len(rows), "weights": "tiny_modernbert/model.safetensors"}

    # seeded 4-layer config with global and local layers
    H, L, NH, I, V = 64, 4, 4, 96, 1000
    shapes = {"embeddings.tok_embeddings.weight": (V, H), "embeddings.norm.weight": (H,),
              "final_norm.weight": (H,)}
    for l in range(L):
        p = f"layers.{l}."
        shapes.update({p + "attn_norm.weight": (H,), p + "attn.Wqkv.weight": (3 * H, H),
                       p + "attn.Wo.weight": (H, H), p + "mlp_norm.weight": (H,),
                       p + "mlp.Wi.weight": (2 * I, H), p + "mlp.Wo.weight": (H, I)})
    w = {}
    for idx, name in enumerate(sorted(shapes)):
        mean, std = synth4_init(name)
        w[name] = O.normal(20261201, 700 + idx, shapes[name], mean, std)
    kw = dict(vocab_size=V, hidden_size=H, num_hidden_layers=L, num_attention_heads=NH, intermediate_size=I,
              pad_token_id=0, bos_token_id=None, eos_token_id=None, cls_token_id=None, sep_token_id=None,
              norm_eps=1e-5, global_attn_every_n_layers=3, local_attention=16, max_position_embeddings=256,
              global_rope_theta=160000.0, local_rope_theta=10000.0)
    rows = [O.uniform_int(20261201, 800 + i, n, 0, V - 1).tolist() for i, n in enumerate([37, 50])]
    hs = run(build(kw, w, True), rows)
    for i, (r, h) in enumerate(zip(rows, hs)):
        out[f"synth4.ids{i}"] = np.asarray(r, np.int32)
        out[f"synth4.hidden{i}"] = h
    cases["synth4"] = {"rows": len(rows), "hidden": H, "layers": L, "heads": NH, "intermediate": I, "vocab": V,
                       "global_every": 3, "local_attention": 16, "global_theta": 160000.0, "local_theta": 10000.0,
                       "weight_seed": 20261201, "weight_stream_base": 700,
                       "init": "norms N(1,0.05), mlp.Wi N(0,0.5), mlp.Wo N(0,0.2), others N(0,0.05)"}
    (HERE / "modernbert").mkdir(exist_ok=True)
    save_file(out, str(HERE / "modernbert" / "vectors.safetensors"))
    (HERE / "modernbert" / "cases.json").write_text(json.dumps(cases, indent=1) + "\n")
    print("wrote", sorted(out))


if __name__ == "__main__":
    main()
