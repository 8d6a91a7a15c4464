"""The C ABI without a GPU: the library loads, exports every symbol include/huncho_rocm.h
declares, fails cleanly when no GPU is visible (the device.rs:34-56 auto-fallback
condition), and its host-side helpers agree with the oracle."""
import re
from pathlib import Path

import numpy as np
import pytest

from huncho_amd import abi
from oracle import oracle as O

HEADER = Path(__file__).resolve().parents[1] / "include" / "huncho_rocm.h"


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hk_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    names = header_functions()
    assert len(names) >= 25
    L = abi.lib()
    for n in names:
        assert hasattr(L, n), f"{n} declared in the header but not exported"
        assert n in abi.SIGNATURES, f"{n} missing from the ctypes binding"
    assert set(abi.SIGNATURES) == set(names)


def test_version_string():
    assert b"gfx950" in abi.lib().hk_version()


def test_context_without_gpu_is_unsupported():
    if abi.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(abi.HkError) as e:
        abi.Context(0)
    assert e.value.code == abi.HK_ERR_UNSUPPORTED


def test_null_context_is_rejected():
    L = abi.lib()
    assert L.hk_ctx_synchronize(None) == abi.HK_ERR_INVALID
    assert L.hk_paged_prefill_attention(None, 0, *([None] + [0] * 2 + [None] * 2 + [0] * 2 + [None, 0] + [None] * 2 +
                                                  [0] * 6 + [0.0, None, 0, 0, None, 0, 0])) == abi.HK_ERR_INVALID


def test_calibrate_matches_oracle_bitwise():
    rng = np.random.default_rng(0)
    for n in (1, 3, 8, 50):
        x = rng.normal(size=n).astype(np.float32) * 4
        for T in (1.0, 1.3, 2.406050072164233):
            assert np.array_equal(abi.calibrate(x, T), O.calibrate(x, T))
    with pytest.raises(abi.HkError):
        abi.calibrate([0.0, float("nan")], 1.0)
    with pytest.raises(abi.HkError):
        abi.calibrate([0.0], -1.0)


def test_synthetic_streams_match_oracle():
    a = abi.synth_normal(1234, 7, 4097, 0.0, 0.02)
    assert np.array_equal(a, O.normal(1234, 7, (4097,), 0.0, 0.02))
    b = abi.synth_normal_bf16(99, 3, 1001)
    assert np.array_equal(b, O.bf16_bits(O.normal(99, 3, (1001,))))
    assert np.array_equal(abi.synth_uniform_int(5, 1, 500, 64, 2048), O.uniform_int(5, 1, 500, 64, 2048))
    assert np.array_equal(abi.synth_permutation(5, 2, 4096), O.permutation(5, 2, 4096))


@pytest.mark.parametrize("rd,theta,bf16", [(128, 1e7, False), (128, 1e7, True), (64, 10000.0, True)])
def test_rope_table_matches_oracle(rd, theta, bf16):
    cs, sn = abi.rope_table(rd, theta, 300, bf16)
    oc, osn = O.rope_cos_sin(rd, theta, np.arange(300), bf16)
    assert np.array_equal(cs, oc[:, : rd // 2]) and np.array_equal(sn, osn[:, : rd // 2])
