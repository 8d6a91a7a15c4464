"""Replicas: model weights staged once per replica from the same host tensors, each replica with
its own context (stream, GEMM plans, workspace), driven concurrently from several host threads.
Every replica's decision logits equal the primary's sequential results bit for bit
(crates/huncho-backend/tests/replicas.rs:8-86, replica() at crates/huncho-api/src/replicas.rs).
"""
import threading

import numpy as np
import pytest
import torch

from huncho_amd import abi
from huncho_amd.kev import KevModel, KevShape, synthetic_weights

pytestmark = pytest.mark.gpu

SEED = 5151
N_REPLICAS = 3
SHAPE = KevShape(hidden=256, n_layers=4, n_heads=2, n_kv_heads=1, intermediate=512, vocab=1000,
                 lin_n_k_heads=2, lin_n_v_heads=2, rotary_dim=64, rope_theta=10000.0, n_out=5)


def _requests():
    lengths = [[70, 129, 1], [300], [64, 64, 65, 17], [2, 511]]
    return [[abi.synth_uniform_int(SEED, 100 * j + i, L, 0, SHAPE.vocab - 1) for i, L in enumerate(ls)]
            for j, ls in enumerate(lengths)]


class Replica:
    """One replica: a context on a stream of its own and a model created from the host weights."""

    def __init__(self, weights, dtype):
        self.stream = torch.cuda.Stream(device=0)
        self.ctx = abi.Context(0, stream=self.stream.cuda_stream)
        with torch.cuda.stream(self.stream):
            self.model = KevModel(self.ctx, SHAPE, weights, dtype)

    def forward(self, rows):
        with torch.cuda.stream(self.stream):
            return self.model.forward_batch(rows)

    def close(self):
        self.model.close()
        self.ctx.close()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_replicas_match_primary_concurrently(dtype):
    weights = synthetic_weights(SHAPE, SEED, std=0.05)
    requests = _requests()
    primary = Replica(weights, dtype)
    expected = [primary.forward(rows) for rows in requests]
    replicas = [Replica(weights, dtype) for _ in range(N_REPLICAS)]
    torch.cuda.synchronize()
    errors = []

    def run(replica, k):
        try:
            for rep in range(2):
                order = list(range(len(requests)))
                if (k + rep) % 2:
                    order.reverse()  # the replicas work on different requests at the same time
                for j in order:
                    logits, probs = replica.forward(requests[j])
                    if not (np.array_equal(logits.view(np.uint32), expected[j][0].view(np.uint32))
                            and np.array_equal(probs, expected[j][1])):
                        errors.append((k, rep, j, float(np.abs(logits - expected[j][0]).max())))
        except Exception as e:  # surfaced after the join
            errors.append((k, repr(e)))

    threads = [threading.Thread(target=run, args=(r, k)) for k, r in enumerate(replicas)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=90)
    assert not any(t.is_alive() for t in threads), "a replica thread did not finish"
    print(f"{dtype}: {N_REPLICAS} replicas x {2 * len(requests)} batches, mismatches: {errors}")
    assert not errors, errors
    for r in replicas + [primary]:
        assert r.ctx.take_faults() == 0
        r.close()
