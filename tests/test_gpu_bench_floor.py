"""The bench-only floor kernels (smith_amd/lib/smith_bench.hsaco through
libsmith_bench.so, outside the product library and its header) that
bench.py times beside the config-1 GEMVs: every kernel runs from a captured
graph on small buffers, returns a positive per-launch time and writes
nothing; an unknown kernel name fails with the helper's error."""
import numpy as np
import pytest

import bench
from smith_amd import device

pytestmark = pytest.mark.gpu


def test_floor_kernels_run_and_write_nothing():
    N = 64
    nbytes = 128 * N * 24
    bufs = [device.alloc(nbytes) for _ in range(2)]
    out = device.alloc(256)
    for b in bufs + [out]:
        device.check(device.lib.smith_fill_zero(device.ops_ctx(), b, 256 if b == out else nbytes))
    device.sync()
    for name, n, grid, block in (("floor_empty", nbytes // 16, 8, 256), ("floor_stream_read", nbytes // 16, 8, 256),
                                 ("floor_block_read", nbytes // 16 - 3, (nbytes // 16 + 767) // 768, 128),
                                 ("floor_q4s_record_read", N, N // 16, 512),
                                 ("floor_q40t_record_read", N, N // 16, 512)):
        us = bench.floor_us(name, bufs, n, out, grid, block, 4)
        assert us > 0, name
    assert not device.download(out, 256, np.uint8).any()
    with pytest.raises(RuntimeError, match="floor kernel"):
        bench.floor_us("no_such_kernel", bufs, 16, out, 1, 64, 1)
    for b in bufs + [out]:
        device.release_buffer(b)


def test_same_grid_record_floors_stay_in_range():
    """The record-read floors of every batched / single-row GEMV variant
    (bench.GEMV_VARIANTS: the kernel's grid, lanes and clamped records) on a
    small weight of each layout: positive times, nothing written."""
    K, N = 1024, 136  # 32 groups; N not a multiple of the 64-column blocks
    G = K // 32
    out = device.alloc(256)
    device.check(device.lib.smith_fill_zero(device.ops_ctx(), out, 256))
    for tag, nbytes in (("q4s", bench.q4s_bytes(K, N)), ("q40t", N // 16 * 16 * G * 18)):
        n_cols = N if tag == "q4s" else N // 16 * 16
        bufs = [device.alloc(nbytes) for _ in range(2)]
        for b in bufs:
            device.check(device.lib.smith_fill_zero(device.ops_ctx(), b, nbytes))
        device.sync()
        for fmt, suffix, threads, grid in bench.GEMV_VARIANTS:
            gx, gy = grid(n_cols, G)
            n = n_cols | (G << 20) | (gx << 40)
            us = bench.floor_us("floor_rec_%s_%s" % (tag, suffix), bufs, n, out, gx * gy, threads, 4)
            assert us > 0, (tag, suffix)
        for b in bufs:
            device.release_buffer(b)
    assert not device.download(out, 256, np.uint8).any()
    device.release_buffer(out)
