"""hk_lora_merge (merge_lora_into_map, crates/huncho-backend/src/qwen3_5.rs:1597-1640) against
the oracle's merge_lora, which the reference's tiny Kev golden vectors pin (dropping it breaks
the golden match: tests/test_oracle.py).

Gates: fp32 merged weights within 1e-6 relative of the oracle's fp32 merge; bf16 merged weights
equal to the oracle's bf16 merge (base weights cast to bf16 at load, the sum cast again, as the
reference loads then merges, qwen3_5.rs:2467-2470, 2283), except for at most 1 bf16 ulp where
the fp32 delta's summation order moves a value across a rounding boundary."""
import json

import numpy as np
import pytest
import torch

from huncho_amd import abi
from huncho_amd.kev import merge_lora_on_device
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from huncho_amd.ops import context_for_torch

    c = context_for_torch(0)
    yield c
    c.close()


def _fixture(golden_dir):
    from safetensors.numpy import load_file

    root = golden_dir / "tiny_kev"
    weights = load_file(str(root / "model.safetensors"))
    lora = load_file(str(root / "adapter_model.safetensors"))
    ac = json.loads((root / "adapter_config.json").read_text())
    return weights, lora, ac["lora_alpha"] / ac["r"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_tiny_kev_lora_merge(ctx, golden_dir, dtype):
    weights, lora, scale = _fixture(golden_dir)
    ref = O.merge_lora(weights, lora, scale, bf16=dtype == torch.bfloat16)
    staged = {k: torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(dtype).cuda() for k, v in weights.items()}
    hk = abi.HK_F32 if dtype == torch.float32 else abi.HK_BF16
    merge_lora_on_device(ctx, staged, lora, scale, hk)
    changed = [k for k in weights if not np.array_equal(ref[k], weights[k])]
    assert len(changed) == 3  # in_proj_qkv of layer 0, gate_proj and q_proj of layer 1
    for k in weights:
        got = staged[k].float().cpu().numpy()
        if dtype == torch.float32:
            e = float(np.abs(got - ref[k]).max() / max(np.abs(ref[k]).max(), 1e-30))
            assert e < 1e-6, (k, e)
        else:
            want = ref[k] if k in changed else O.round_bf16(ref[k])
            ulp = np.abs(O.bf16_bits(got).astype(np.int32) - O.bf16_bits(want).astype(np.int32))
            assert ulp.max() <= 1, (k, int(ulp.max()))


def test_lora_merge_large_rank(ctx):
    """A 512 x 1024 bf16 weight with a rank-16 adapter against a float64 merge."""
    rows, cols, r, scale = 512, 1024, 16, 2.0
    w = O.round_bf16(abi.synth_normal(5, 1, rows * cols, 0.0, 0.02)).reshape(rows, cols)
    a = abi.synth_normal(5, 2, r * cols, 0.0, 0.1).reshape(r, cols)
    b = abi.synth_normal(5, 3, rows * r, 0.0, 0.1).reshape(rows, r)
    wd = torch.from_numpy(w).to(torch.bfloat16).cuda()
    ad, bd = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    ctx.check(abi.lib().hk_lora_merge(ctx.h, abi.HK_BF16, wd.data_ptr(), rows, cols, ad.data_ptr(), bd.data_ptr(),
                                      r, scale))
    torch.cuda.synchronize()
    ref = w.astype(np.float64) + scale * (b.astype(np.float64) @ a.astype(np.float64))
    got = wd.float().cpu().numpy()
    # within half a bf16 ulp of the exact sum, plus the fp32 delta's own rounding
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6)
    with pytest.raises(abi.HkError):
        ctx.check(abi.lib().hk_lora_merge(ctx.h, abi.HK_BF16, wd.data_ptr(), rows, cols, ad.data_ptr(),
                                          bd.data_ptr(), 0, scale))
