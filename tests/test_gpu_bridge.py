"""GPU tests of the reference bridge entries beyond begin / dispatch /
end_sync (native/gpu_bridge.h:26-127, as src/device.js:10-50 binds them and
src/dispatch.js:17-48 / src/profile.js:35-55 use them): device limits,
hipRTC compilation (smith_compile_source), dynamic LDS
(smith_set_threadgroup_memory), timed / asynchronous / one-shot dispatch,
and the release self-tests."""
import ctypes

import numpy as np
import pytest

from smith_amd import device, dispatch, prng

pytestmark = pytest.mark.gpu

# y[i] = a[n-1-i within the group] * s + a[i]: the reversal goes through
# dynamic LDS, so a missing or short threadgroup-memory block shows up
SRC = r'''
extern "C" __global__ void smith_rtc_mirror(float* out, const float* a, float s, unsigned n) {
  extern __shared__ float sm[];
  const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  sm[threadIdx.x] = i < n ? a[i] : 0.f;
  __syncthreads();
  if (i < n) out[i] = sm[blockDim.x - 1 - threadIdx.x] * s + sm[threadIdx.x];
}
'''


def _expect(a, s, group):
    n = a.size
    pad = np.zeros(-(-n // group) * group, np.float32)
    pad[:n] = a
    rev = pad.reshape(-1, group)[:, ::-1].ravel()[:n]
    return (rev * np.float32(s) + a).astype(np.float32)


@pytest.fixture(scope="module")
def rtc():
    lib_ = device.compile_source(SRC)
    return device.create_pipeline(lib_, "smith_rtc_mirror")


def test_device_limits():
    c = device.ctx()
    assert device.lib.smith_max_threads_per_threadgroup(c) == 1024
    lds = device.lib.smith_max_threadgroup_memory(c)
    assert lds >= 64 * 1024 and lds % 1024 == 0, lds
    assert "gfx950" in device.device_name()


def test_release_self_tests():
    # src/device.js:62-63 expects ~1048576 bytes freed by both
    c = device.ctx()
    assert device.lib.smith_test_release(c) == 1 << 20
    assert device.lib.smith_test_release_after_use(c) == 1 << 20
    b = device.alloc(1000)
    assert device.lib.smith_buffer_retain_count(b) == 1 and device.lib.smith_buffer_length(b) == 1000
    before = device.lib.smith_allocated_size(c)
    device.release_buffer(b)
    assert device.lib.smith_allocated_size(c) == before - 1000
    assert device.lib.smith_buffer_retain_count(b) == 0


def _buffers(n, seed):
    a = prng.randn((n,), seed)
    ba, bo = device.alloc(n * 4), device.alloc(n * 4)
    device.upload(ba, a)
    return a, ba, bo


@pytest.mark.parametrize("n,group", [(1000, 256), (64, 64), (4097, 128)])
def test_compile_source_dynamic_lds_end_timed(rtc, n, group):
    """hipRTC kernel, dynamic LDS of group floats, Metal dispatchThreads grid
    (n threads, ragged last group), timed completion as dispatch.run's
    profiling path records it (smith_end_timed)."""
    a, ba, bo = _buffers(n, 70 + n)
    enc = device.begin()
    device.set_pipeline(enc, rtc)
    device.set_buffer(enc, bo, 0)
    device.set_buffer(enc, ba, 1)
    device.set_bytes(enc, np.float32(0.5).tobytes(), 2)
    device.set_bytes(enc, np.uint32(n).tobytes(), 3)
    device.set_threadgroup_memory(enc, group * 4, 0)
    device.dispatch(enc, n, 1, 1, group, 1, 1)
    t = device.end_timed(enc)
    assert t["gpuMs"] > 0 and t["gpuEnd"] >= t["gpuStart"] > 0
    assert np.array_equal(device.download(bo, n * 4, np.float32), _expect(a, 0.5, group))


def test_dispatch_run_profiling_records_time():
    """dispatch.run with profiling on (src/dispatch.js:42-47) goes through
    smith_end_timed: the reference-bound matmul_q8 kernel, its count and
    time recorded, the result unchanged."""
    from oracle import oracle as O
    K, N, M = 96, 40, 2
    w = prng.randn((K, N), 84, std=0.02)
    a = prng.randn((M, K), 85)
    q = O.quantize_q8(w)
    bq, ba, bc = device.alloc(q.nbytes), device.alloc(a.nbytes), device.alloc(M * N * 4)
    device.upload(bq, q)
    device.upload(ba, a)
    params = np.array([M, N, K, K // 32], np.uint32).tobytes()
    dispatch.enable_profiling(True)
    try:
        for _ in range(3):
            dispatch.run("matmul_q8", [{"buffer": ba, "index": 0}, {"buffer": bq, "index": 1},
                                       {"buffer": bc, "index": 2}],
                         {"x": N, "y": M}, {"x": 16, "y": 16}, {"data": params, "index": 3})
        rep = dispatch.report()
    finally:
        dispatch.enable_profiling(False)
    assert rep["matmul_q8"]["count"] == 3 and rep["matmul_q8"]["totalMs"] > 0.0
    want = O.matmul_q8(a, q, K, N)
    got = device.download(bc, M * N * 4, np.float32).reshape(M, N)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


def test_end_async_and_wait(rtc):
    n, group = 3000, 256
    a, ba, bo = _buffers(n, 81)
    enc = device.begin()
    device.set_pipeline(enc, rtc)
    device.set_buffer(enc, bo, 0)
    device.set_buffer(enc, ba, 1)
    device.set_bytes(enc, np.float32(-2.0).tobytes(), 2)
    device.set_bytes(enc, np.uint32(n).tobytes(), 3)
    device.set_threadgroup_memory(enc, group * 4, 0)
    device.dispatch(enc, n, 1, 1, group, 1, 1)
    token = device.end_async(enc)
    assert token
    device.wait(token)
    assert np.array_equal(device.download(bo, n * 4, np.float32), _expect(a, -2.0, group))


def test_dispatch_sync_one_shot():
    """smith_dispatch_sync (gpu_bridge.h:101-110) on a code-object kernel:
    the reference-semantics matmul_q8 with buffers and params by index."""
    from oracle import oracle as O
    K, N, M = 64, 48, 3
    w = prng.randn((K, N), 82, std=0.02)
    a = prng.randn((M, K), 83)
    q = O.quantize_q8(w)
    bq, ba, bc = device.alloc(q.nbytes), device.alloc(a.nbytes), device.alloc(M * N * 4)
    device.upload(bq, q)
    device.upload(ba, a)
    bufs = (ctypes.c_void_p * 3)(ba, bq, bc)
    idx = (ctypes.c_uint32 * 3)(0, 1, 2)
    params = np.array([M, N, K, K // 32], np.uint32)
    device.lib.smith_dispatch_sync(device.ctx(), device.pipeline("matmul_q8"), bufs, idx, 3,
                                   params.ctypes.data_as(ctypes.c_void_p), params.nbytes, 3, N, M, 1, 16, 16, 1)
    got = device.download(bc, M * N * 4, np.float32).reshape(M, N)
    want = O.matmul_q8(a, q, K, N)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


def test_compile_source_error_is_reported():
    with pytest.raises(RuntimeError, match="shader compilation failed"):
        device.compile_source('extern "C" __global__ void broken(float* o) { o[0] = undefined_name; }')


def _fresh_ctx():
    c = device.lib.smith_init()
    assert c
    for path in (device.CODE_OBJECT_PATH, device.LLAMA_CODE_OBJECT_PATH, device.GEMM_CODE_OBJECT_PATH):
        assert device.lib.smith_load_library(c, path.encode()), device.lib.smith_last_error(c)
    return c


def test_first_split_k_calls_on_a_fresh_context():
    """The split-K counters a context allocates on first use are zeroed on
    its own stream before the first kernel reads them (zeroed on the null
    stream, which the context's stream is not ordered after, the first
    Q6_K LM head of a fresh process returned garbage, and the counters it
    left behind broke every later call).  On a new context the very first
    split-K launches -- a Q6_K LM head (12 K splits) on one context, a
    single-row GEMV split across blocks (K = 14336) on another -- match the
    oracle."""
    from oracle import oracle as O
    lib = device.lib
    K, N = 3072, 4096
    w = prng.randn((K, N), 71, std=0.02)
    x = prng.randn((K,), 72)
    c = _fresh_ctx()
    try:
        blocks = O.quantize_rows(O.GGML_Q6_K, w)
        wd = O.dequantize_tensor(O.GGML_Q6_K, blocks, K * N).reshape(K, N).astype(np.float64)
        src = device.alloc(blocks.nbytes)
        device.upload(src, blocks)
        planes = device.alloc(int(lib.smith_lmhead_q6_k_bytes(K, N)))
        xb, yb = device.alloc(K * 4), device.alloc(N * 4)
        device.upload(xb, x.astype(np.float32))
        assert lib.smith_repack_lmhead_q6_k(c, src, planes, K, N) == 0
        assert lib.smith_lmhead_q6_k_nb(c, xb, None, 0.0, planes, yb, K, N) == 0
        assert lib.smith_sync(c) == 0
        y = device.download(yb, N * 4, np.float32)
        assert O.normwise_rel_err(y, x.astype(np.float64) @ wd) <= 2e-6
        for b in (src, planes, xb, yb):
            device.release_buffer(b)
    finally:
        lib.smith_destroy(c)
    c = _fresh_ctx()
    try:
        Kg, Ng = 14336, 4096
        wg = prng.randn((Kg, Ng), 73, std=0.02)
        a = prng.randn((1, Kg), 74)
        q = O.quantize_q4s(wg)
        qb, ab, ob = device.alloc(q.nbytes), device.alloc(a.nbytes), device.alloc(Ng * 4)
        device.upload(qb, q)
        device.upload(ab, a)
        assert lib.smith_matmul_q4(c, ab, qb, ob, 1, Ng, Kg, Kg // 32) == 0
        assert lib.smith_sync(c) == 0
        y = device.download(ob, Ng * 4, np.float32)
        assert O.normwise_rel_err(y, O.matmul_q4s(a, q, Kg, Ng)) <= 2e-5
        for b in (qb, ab, ob):
            device.release_buffer(b)
    finally:
        lib.smith_destroy(c)
