"""smith_matmul_q4_noalloc (static device scratch, no allocation) against
smith_matmul_q4 through the C ABI: bit-identical outputs (same kernels, same
fixed split-K order) on consecutive calls -- the second with a smaller input
-- on the decode paths that use each scratch region, and a clear error for a
shape whose scratch exceeds the static array."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from smith_amd import device, prng

pytestmark = pytest.mark.gpu


def _run(fn, a_buf, q_buf, M, N, K):
    out = device.alloc(M * N * 4)
    rc = fn(device.ops_ctx(), a_buf, q_buf, out, M, N, K, (K + 31) // 32)
    device.check(rc, fn.__name__)
    y = device.download(out, M * N * 4, np.float32).reshape(M, N)
    device.release_buffer(out)
    return y


# (M, N, K): M=1 with a cross-block K split (partials + counters), M=4 / 8
# (one-launch GEMV with K splits), M=16 / 32 (activation staging + partials),
# M=64 (f16 staging of the GEMM); each pair: second call smaller
CASES = [((1, 4096, 14336), (1, 1024, 4096)), ((8, 4096, 4096), (4, 1024, 2048)),
         ((32, 4096, 4096), (16, 2048, 4096)), ((64, 1024, 4096), (64, 512, 1024))]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_allocating_entry(first, second):
    lib = device.lib
    for i, (M, N, K) in enumerate((first, second)):
        print("noalloc case", M, N, K, flush=True)
        w = prng.randn((K, N), 900 + i + M, std=0.02)
        a = prng.randn((M, K), 950 + i + M)
        q = O.quantize_q4s(w)
        bq, ba = device.alloc(q.nbytes), device.alloc(a.nbytes)
        device.upload(bq, q)
        device.upload(ba, a)
        want = _run(lib.smith_matmul_q4, ba, bq, M, N, K)
        before = lib.smith_allocated_size(device.ctx())
        got = _run(lib.smith_matmul_q4_noalloc, ba, bq, M, N, K)
        got2 = _run(lib.smith_matmul_q4_noalloc, ba, bq, M, N, K)  # counters left at zero by the first
        assert lib.smith_allocated_size(device.ctx()) == before
        assert np.array_equal(got, want) and np.array_equal(got2, want), (M, N, K)
        assert O.normwise_rel_err(got, O.matmul_q4s(a, q, K, N)) <= 1e-3
        device.release_buffer(bq)
        device.release_buffer(ba)


def test_noalloc_rejects_oversized_scratch():
    """M = 512 at K = 14336 needs 14.7 MB of f16 activation staging, beyond
    the 4 MiB region: -1 and a message naming the sizes, nothing launched."""
    M, N, K = 512, 1024, 14336
    q = np.zeros((K // 32) * N * 24, np.uint8)
    bq, ba, bo = device.alloc(q.nbytes), device.alloc(M * K * 4), device.alloc(M * N * 4)
    rc = device.lib.smith_matmul_q4_noalloc(device.ops_ctx(), ba, bq, bo, M, N, K, K // 32)
    assert rc == -1
    msg = device.lib.smith_last_error(device.ctx()).decode()
    assert "smith_matmul_q4_noalloc" in msg and "static scratch" in msg, msg
    device.sync()
    for b in (bq, ba, bo):
        device.release_buffer(b)
