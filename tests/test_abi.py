"""C-ABI boundary checks that need no GPU: the library loads, exports every
symbol include/smith.h declares, the code object holds every kernel the
bridge launches, and host-side errors match the reference's messages."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "smith.h")


def declared_symbols():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(smith_\w+)\s*\(", src)))


def test_library_exports_header_symbols():
    from smith_amd import device
    names = declared_symbols()
    assert len(names) >= 40
    for n in names:
        assert hasattr(device.lib, n), n
        assert n in device.SYMBOLS, "ctypes table lacks " + n
    assert set(device.SYMBOLS) == set(names)


def test_reference_bridge_names_all_present():
    # the 25 functions of native/gpu_bridge.h:15-127, bound at src/device.js:10-50
    ref = ["smith_init", "smith_destroy", "smith_device_name", "smith_max_threadgroup_memory",
           "smith_max_threads_per_threadgroup", "smith_alloc", "smith_buffer_contents", "smith_buffer_length",
           "smith_release_buffer", "smith_load_library", "smith_compile_source", "smith_create_pipeline",
           "smith_begin", "smith_set_buffer", "smith_set_bytes", "smith_set_threadgroup_memory",
           "smith_set_pipeline", "smith_dispatch", "smith_end_sync", "smith_end_async", "smith_wait",
           "smith_end_timed", "smith_allocated_size", "smith_test_release", "smith_test_release_after_use",
           "smith_buffer_retain_count", "smith_dispatch_sync"]
    assert set(ref) <= set(declared_symbols())


def test_code_object_has_kernels():
    from smith_amd import device
    out = subprocess.run(["/opt/rocm/llvm/bin/llvm-readelf", "--syms", device.CODE_OBJECT_PATH],
                         capture_output=True, text=True, check=True).stdout
    need = ["matmul_q4", "matmul_q8", "smith_quantize_q4s", "smith_quantize_q8", "smith_quantize_q4_0_rows",
            "smith_repack_q4_0_cols", "smith_repack_q8_0_cols", "smith_repack_q4_0_tiles", "smith_zero_u32"]
    for fmt in ("q4", "q8", "q40"):
        need += ["smith_qprep_%s_hilo" % fmt, "smith_qprep_%s_plain" % fmt]
    for fmt in ("q40t", "q41t", "q50t", "q4kt", "q6kt"):
        need += ["smith_agemv_%s_k%d" % (fmt, k) for k in (32, 48, 64, 72, 96, 128, 144, 192, 288)]
        need += ["smith_agemv_att_%s_k%d" % (fmt, k) for k in (64, 96, 128, 192)]
    for fmt in ("q4s", "q8", "q40", "q40t"):
        need += ["smith_qgemv3_%s_m%d" % (fmt, m) for m in (4, 8, 16, 32)]
        need += ["smith_qgemv1_%s_m%d_k%d" % (fmt, m, k) for m in (1, 2) for k in (64, 96, 128, 288)]
        need += ["smith_qgemv1_%s_m1_k%d_c2" % (fmt, k) for k in (96, 128)]
        need += ["smith_qgemv1_%s_m1_k448w16_pl" % fmt]
        # every variant qgemv5_chunk can name (bucket x shape)
        need += ["smith_qgemv5_%s_m%d_%s" % (fmt, m, v) for m in (4, 8, 16, 32) for v in ("w16", "k32", "k32c4")
                 if not (m == 32 and v == "w16")]
        need += ["smith_qgemv5_%s_m32_k64c2" % fmt]
    need += ["smith_qgemv1_q8c_m1_k%d_pl" % k for k in (64, 96, 128, 288)]
    need += ["smith_qgemv1_q8c_m1_k%d_c2_pl" % k for k in (96, 128)]
    for k in need:
        assert re.search(r"\b%s\.kd\b" % k, out), k
    out = subprocess.run(["/opt/rocm/llvm/bin/llvm-readelf", "--syms", device.GEMM_CODE_OBJECT_PATH],
                         capture_output=True, text=True, check=True).stdout
    for k in ["smith_gemm_prep_a", "smith_gemm_prep_a_perm", "smith_gemm_reduce"] + [
            "smith_gemm_%s_m%d_n%d" % (f, m, n) for f in ("q4s", "q8", "q40", "q40t", "q41t", "q50t", "q4kt", "q6kt")
            for (m, n) in ((128, 64), (128, 128), (256, 128), (256, 256))] + [
            "smith_gemm2_%s_m%d_n%d" % (f, m, n) for f in ("q40t", "q41t", "q50t", "q4kt", "q6kt")
            for (m, n) in ((128, 64), (128, 128), (256, 128), (256, 256))]:
        assert re.search(r"\b%s\.kd\b" % k, out), k
    out = subprocess.run(["/opt/rocm/llvm/bin/llvm-readelf", "--syms", device.LLAMA_CODE_OBJECT_PATH],
                         capture_output=True, text=True, check=True).stdout
    for k in ["smith_rmsnorm_rows", "smith_embed_rows", "smith_attention", "smith_attention_part", "smith_kv_append", "smith_attention_cached",
              "smith_lmhead_q4_0_nb", "smith_repack_lmhead_q4_0", "smith_lmhead_q6_k_nb", "smith_repack_lmhead_q6_k",
              "smith_gemv_f32_kn", "smith_gemv_f32_nk", "smith_argmax_embed", "smith_set_i32", "smith_randn_f32"] + [
              "smith_repack_gt_%s" % f for f in ("q40", "q41", "q50", "q4k", "q6k")] + [
              "smith_attention_prefill_hd%d" % n for n in range(1, 9)] + [
              "smith_dequantize_%s" % t for t in ("f16", "bf16", "q4_0", "q4_1", "q5_0", "q8_0", "q4_k", "q6_k")]:
        assert re.search(r"\b%s\.kd\b" % k, out), k


def test_package_imports_without_gpu_and_errors_match_reference():
    import smith_amd

    class FakeA:
        shape = [1, 48]
        dtype = "f32"
        buffer = None

    wq = smith_amd.QuantizedWeight(buffer=None, K=64, N=8, groups=2, totalBytes=2 * 8 * 24)
    with pytest.raises(ValueError, match="matmulQ4: inner dims don't match: 48 vs 64"):
        smith_amd.matmulQ4(FakeA(), wq)
    with pytest.raises(ValueError, match="matmulQ8: inner dims don't match: 48 vs 64"):
        smith_amd.matmulQ8(FakeA(), wq)
