"""Build the gfx950 code object and the C-ABI bridge in-tree.

  smith_amd/lib/smith_kernels.hsaco   hipcc --offload-device-only --offload-arch=gfx950
  smith_amd/lib/smith_llama.hsaco     (the GGUF decode-path kernels, same flags)
  smith_amd/lib/smith_gemm.hsaco      (the prefill MFMA GEMM, same flags)
  smith_amd/lib/libsmith.so           hipcc -x hip: host code against libamdhip64 (+ static device scratch)
  smith_amd/lib/smith_bench.hsaco     bench-only floor kernels (bench_floor.hip)
  smith_amd/lib/libsmith_bench.so     bench-only host helper that times them (bench_floor_host.cpp)

Run as `python -m smith_amd.build`; __graft_entry__.build() calls build().
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HSACO = os.path.join(LIBDIR, "smith_kernels.hsaco")
HSACO_LLAMA = os.path.join(LIBDIR, "smith_llama.hsaco")
HSACO_GEMM = os.path.join(LIBDIR, "smith_gemm.hsaco")
LIBSMITH = os.path.join(LIBDIR, "libsmith.so")
# bench-only: the floor kernels bench.py times beside the product's steps
HSACO_BENCH = os.path.join(LIBDIR, "smith_bench.hsaco")
LIBBENCH = os.path.join(LIBDIR, "libsmith_bench.so")

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (unreliable on the pool).
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.check_call(cmd)


def _kernel_cmds():
    # a plain gfx950 ELF code object (no offload bundle) for hipModuleLoad
    return [[os.path.join(ROCM, "bin", "hipcc"), *HIP_FLAGS, "--offload-device-only", "--no-gpu-bundle-output",
             "-c", os.path.join(CSRC, src), "-o", dst]
            for src, dst in (("smith_kernels.hip", HSACO), ("llama_kernels.hip", HSACO_LLAMA),
                             ("gemm_kernels.hip", HSACO_GEMM), ("bench_floor.hip", HSACO_BENCH))]


def _bridge_cmd():
    # compiled as HIP: besides the host code it holds the static device
    # scratch of smith_matmul_q4_noalloc (a gfx950 code object with no kernels)
    return [os.path.join(ROCM, "bin", "hipcc"), "-x", "hip", *HIP_FLAGS, "-fPIC", "-shared", "-Wall",
            "-Wno-unused-result", "-Wno-unused-value", "-I" + os.path.join(ROCM, "include"),
            os.path.join(CSRC, "smith_bridge.cpp"), "-o", LIBSMITH,
            "-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-lhiprtc",
            "-Wl,-rpath," + os.path.join(ROCM, "lib")]


def _bench_cmd():
    return [os.path.join(ROCM, "bin", "hipcc"), "-x", "hip", *HIP_FLAGS, "-fPIC", "-shared", "-Wall",
            "--offload-host-only", os.path.join(CSRC, "bench_floor_host.cpp"), "-o", LIBBENCH,
            "-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib")]


def build_kernels():
    os.makedirs(LIBDIR, exist_ok=True)
    for cmd in _kernel_cmds():
        _run(cmd)


def build_bridge():
    os.makedirs(LIBDIR, exist_ok=True)
    _run(_bridge_cmd())


def build():
    """Every code object and the bridge, compiled concurrently (independent
    translation units); fails if any of them fails."""
    os.makedirs(LIBDIR, exist_ok=True)
    cmds = _kernel_cmds() + [_bridge_cmd(), _bench_cmd()]
    procs = []
    for cmd in cmds:
        print("+", " ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd)))
    bad = [cmd for cmd, p in procs if p.wait() != 0]
    if bad:
        raise subprocess.CalledProcessError(1, bad[0])


if __name__ == "__main__":
    build()
    sys.exit(0)
