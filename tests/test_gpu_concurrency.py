"""Calls from several host threads on their own streams.

The reference's engine drives one device from one thread (engine/fast/model.py:294), and TP
runs one host thread per device (engine/fast/tp.py:903); a library on a shared device must
still give every caller its own results when calls overlap. The prefill-sized block forks
the shared expert onto the library's auxiliary stream, one per device, under a lock held
from the fork to the join; these tests run block calls from two threads, each on its own
stream, and compare every result with the same call made alone."""

from __future__ import annotations

import threading

import pytest
import torch

from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


@pytest.fixture(scope="module")
def mlp(dev):
    import __graft_entry__

    return __graft_entry__._mlp_from_weights(orc.make_weights(2048, 256, 512, 512, seed=41), dev)


@pytest.mark.parametrize("T", [1, 64, 700])
def test_two_threads_on_two_streams_match_serial_calls(pkg, dev, mlp, T):
    print(f"concurrent block calls T={T}", flush=True)
    g = torch.Generator().manual_seed(T)
    xs = [[torch.randn(T, 2048, generator=g).to(BF16).to(dev) for _ in range(4)] for _ in range(2)]
    want = [[pkg.block.moe(x, mlp, 8) for x in row] for row in xs]
    torch.cuda.synchronize()
    got = [[None] * 4 for _ in range(2)]
    errors = []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for rep in range(3):
                    for j, x in enumerate(xs[i]):
                        got[i][j] = pkg.block.moe(x, mlp, 8)
            s.synchronize()
        except Exception as exc:  # pragma: no cover - reported below
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(2):
        for j in range(4):
            assert torch.equal(got[i][j], want[i][j]), (i, j)
