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


def _run(fn, a_buf, q_buf, M, N, K, out=None, ctx=None):
    own = out is None
    if own:
        out = device.alloc(M * N * 4)
    rc = fn(ctx or device.ops_ctx(), a_buf, q_buf, out, M, N, K, (K + 31) // 32)
    device.check(rc, fn.__name__)
    if ctx:
        assert device.lib.smith_sync(ctx) == 0
    else:
        device.sync()
    y = device.download(out, M * N * 4, np.float32).reshape(M, N)
    if own:
        device.release_buffer(out)
    return y


def _fresh_ctx():
    """A second context with the code objects loaded and no op scratch yet."""
    lib = device.lib
    c = lib.smith_init()
    assert c
    for path in (device.CODE_OBJECT_PATH, device.LLAMA_CODE_OBJECT_PATH, device.GEMM_CODE_OBJECT_PATH):
        assert lib.smith_load_library(c, path.encode()), lib.smith_last_error(c)
    return c


def test_noalloc_first_call_on_fresh_context():
    """On a context that has never run an op (no scratch of its own), the
    no-alloc entry point works for shapes that use every region, its
    allocated size stays zero, and a following allocating call agrees."""
    lib = device.lib
    c = _fresh_ctx()
    try:
        assert lib.smith_allocated_size(c) == 0
        # (1, 2048, 14336): a 4-way K split (a 4096-column output covers K in one block)
        for (M, N, K) in ((1, 2048, 14336), (32, 4096, 4096), (64, 1024, 4096)):
            print("noalloc fresh ctx", M, N, K, flush=True)
            w = prng.randn((K, N), 960 + M, std=0.02)
            a = prng.randn((M, K), 970 + M)
            q = O.quantize_q4s(w)
            bq, ba, bo = device.alloc(q.nbytes), device.alloc(a.nbytes), device.alloc(M * N * 4)
            device.upload(bq, q)
            device.upload(ba, a)
            got = _run(lib.smith_matmul_q4_noalloc, ba, bq, M, N, K, bo, ctx=c)
            assert lib.smith_sync(c) == 0
            assert lib.smith_allocated_size(c) == 0
            want = _run(lib.smith_matmul_q4, ba, bq, M, N, K, bo, ctx=c)
            assert lib.smith_sync(c) == 0
            assert lib.smith_allocated_size(c) > 0  # the allocating entry grew its scratch
            assert np.array_equal(got, want), (M, N, K)
            for b in (bq, ba, bo):
                device.release_buffer(b)
            lib.smith_destroy(c)
            c = _fresh_ctx()
    finally:
        lib.smith_destroy(c)


def test_noalloc_ignores_prepared_operand_hint():
    """A hinted K-split GEMM (smith_prep_next) leaves its output rows prepared
    as f16 in the context's own buffer; a no-alloc call on those rows right
    after must prepare its operand in the static array itself, and equals
    smith_matmul_q4 on the same rows."""
    lib = device.lib
    ctx = device.ops_ctx()
    M, D = 128, 1024
    x = prng.randn((M, D), 981)
    res = prng.randn((M, D), 982)
    wt = prng.randn((D, D), 983, std=0.02)  # GGUF listing [out, in]
    xb, rb = device.alloc(x.nbytes), device.alloc(res.nbytes)
    device.upload(xb, x)
    device.upload(rb, res)
    wtb = device.alloc(wt.nbytes)
    device.upload(wtb, wt)
    G = D // 32
    blocks, nib, dsc = device.alloc(D * G * 18), device.alloc(D * G * 16), device.alloc(D * G * 2)
    device.check(lib.smith_quantize_q4_0(ctx, wtb, blocks, D, D))
    device.check(lib.smith_repack_q4_0_t_into(ctx, blocks, nib, dsc, D, D, 0, 1, D))
    w2 = prng.randn((D, 512), 984, std=0.02)
    q2 = O.quantize_q4s(w2)
    bq = device.alloc(q2.nbytes)
    device.upload(bq, q2)
    y1 = device.alloc(M * D * 4)

    def hinted_linear():
        device.check(lib.smith_prep_next(ctx, None, 0.0))
        device.check(lib.smith_linear_q4_0_t(ctx, xb, nib, dsc, y1, M, D, D, None, 0.0, rb, 1))

    hinted_linear()
    got = _run(lib.smith_matmul_q4_noalloc, y1, bq, M, 512, D)
    hinted_linear()
    want = _run(lib.smith_matmul_q4, y1, bq, M, 512, D)
    assert np.array_equal(got, want)
    y1h = device.download(y1, M * D * 4, np.float32).reshape(M, D)
    assert O.normwise_rel_err(got, O.matmul_q4s(y1h, q2, D, 512)) <= 1e-2
    for b in (xb, rb, wtb, blocks, nib, dsc, bq, y1):
        device.release_buffer(b)


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
        # the allocating entry point's scratch counts in the allocated size,
        # so an allocation inside the no-alloc calls would show here
        out = device.alloc(M * N * 4)
        before = lib.smith_allocated_size(device.ctx())
        got = _run(lib.smith_matmul_q4_noalloc, ba, bq, M, N, K, out)
        got2 = _run(lib.smith_matmul_q4_noalloc, ba, bq, M, N, K, out)  # counters left at zero by the first
        assert lib.smith_allocated_size(device.ctx()) == before
        device.release_buffer(out)
        want = _run(lib.smith_matmul_q4, ba, bq, M, N, K)
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
