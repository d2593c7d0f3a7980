"""A captured graph keeps working after the context's scratch grows.

Ops size their scratch (split-K partials, counters, f16 activations) on
first use and grow it when a bigger op comes along.  A HIP graph captured
earlier names the old buffers, so the bridge keeps replaced scratch alive
until the context is destroyed: a replay after the growth must still give
the eager result, bit for bit (same kernels, fixed split-K summation order).
"""
import numpy as np
import pytest

from smith_amd import device, prng
import smith_amd as S

pytestmark = pytest.mark.gpu


def _fresh_ctx():
    c = device.lib.smith_init()
    assert c
    for path in (device.CODE_OBJECT_PATH, device.LLAMA_CODE_OBJECT_PATH, device.GEMM_CODE_OBJECT_PATH):
        assert device.lib.smith_load_library(c, path.encode()), device.lib.smith_last_error(c)
    return c


def test_graph_replay_after_scratch_growth():
    c = _fresh_ctx()
    try:
        M, K, N = 4, 4096, 1024  # the M <= 8 GEMV: K split across workgroups, partials in scratch
        G = K // 32
        w = S.quantizeQ4(S.tensor(prng.randn((K, N), 81, std=0.02)))
        a = S.tensor(prng.randn((M, K), 82))
        ref, got = S.create([M, N]), S.create([M, N])
        device.sync()  # inputs were made on the main context's stream
        device.check(device.lib.smith_matmul_q4(c, a.buffer, w["buffer"], ref.buffer, M, N, K, G))
        device.check(device.lib.smith_sync(c))
        device.check(device.lib.smith_graph_begin(c), "graph begin")
        rc = device.lib.smith_matmul_q4(c, a.buffer, w["buffer"], got.buffer, M, N, K, G)
        g = device.lib.smith_graph_end(c)
        device.check(rc, "captured matmul")
        assert g
        try:
            # a prefill-sized GEMM grows the split-K scratch and the f16 activations
            M2, K2, N2 = 512, 14336, 4096
            w2 = S.quantizeQ4(S.tensor(prng.randn((K2, N2), 83, std=0.02)))
            a2 = S.tensor(prng.randn((M2, K2), 84))
            o2 = S.create([M2, N2])
            device.sync()
            device.check(device.lib.smith_matmul_q4(c, a2.buffer, w2["buffer"], o2.buffer, M2, N2, K2, K2 // 32))
            device.check(device.lib.smith_sync(c))
            # fresh allocations that may land where freed scratch was, filled with junk
            junk = [device.alloc(1 << 22) for _ in range(8)]
            for j in junk:
                device.upload(j, np.full(1 << 20, np.nan, np.float32))
            device.upload(got.buffer, np.zeros((M, N), np.float32))
            device.sync()
            for rep in range(2):
                device.check(device.lib.smith_graph_launch(c, g), "graph launch")
                device.check(device.lib.smith_sync(c))
                out = device.download(got.buffer, M * N * 4, np.float32)
                want = device.download(ref.buffer, M * N * 4, np.float32)
                assert np.array_equal(out, want), rep
            for j in junk:
                device.release_buffer(j)
        finally:
            device.lib.smith_graph_destroy(g)
    finally:
        device.lib.smith_sync(c)
        device.lib.smith_destroy(c)
