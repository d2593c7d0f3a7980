/*
 * smith.h -- C ABI of libsmith.so, the MI355X (gfx950) HIP bridge that
 * replaces SMITH's Objective-C Metal bridge (native/gpu_bridge.h) for the
 * quantized-weight matmul path.
 *
 * Plain C types only: opaque handles are void*, buffers are device pointers
 * returned by smith_alloc (any device pointer inside such a buffer may be
 * passed where a buffer is expected), sizes are uint64_t / uint32_t.
 * One context = one HIP device + one HIP stream (default priority); every
 * launch is enqueued on that stream in call order.
 *
 * Error convention: functions returning a pointer return NULL on failure;
 * functions returning int return 0 on success and a negative code on
 * failure.  smith_last_error(ctx) gives the message of the last failure.
 */
#ifndef SMITH_H
#define SMITH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage modes (native/gpu_bridge.h:12-13).  Both allocate device memory
 * (hipMalloc); SHARED is accepted for API compatibility but is NOT host
 * visible: use smith_copy_h2d / smith_copy_d2h. */
#define SMITH_SHARED 0
#define SMITH_PRIVATE 1

typedef struct SmithEncoder SmithEncoder;

/* Timing of a timed dispatch (native/gpu_bridge.h:113-117).  gpu_start /
 * gpu_end are seconds on the host's steady clock at submit / completion;
 * gpu_ms is the HIP-event duration of the encoded work.  Free with
 * smith_free. */
typedef struct {
  double gpu_start;
  double gpu_end;
  double gpu_ms;
} SmithTiming;

/* ---- lifecycle (gpu_bridge.h:18,21) ---- */
void* smith_init(void);
void smith_destroy(void* ctx);

/* ---- device info (gpu_bridge.h:26-32) ---- */
char* smith_device_name(void* ctx);                    /* free with smith_free */
uint64_t smith_max_threadgroup_memory(void* ctx);      /* LDS bytes per workgroup */
uint64_t smith_max_threads_per_threadgroup(void* ctx);

/* ---- buffers (gpu_bridge.h:37-52) ---- */
void* smith_alloc(void* ctx, uint64_t bytes, uint32_t mode);
void* smith_buffer_contents(void* buffer);  /* always NULL: device memory is not host-mapped */
uint64_t smith_buffer_length(void* buffer); /* 0 for a pointer not returned by smith_alloc */
void smith_release_buffer(void* buffer);
int64_t smith_test_release(void* ctx);
int64_t smith_test_release_after_use(void* ctx);
int64_t smith_buffer_retain_count(void* buffer); /* 1 while live, 0 otherwise */
uint64_t smith_allocated_size(void* ctx);

/* ---- explicit copies (new: replace Metal's shared-memory zero copy) ---- */
int smith_copy_h2d(void* ctx, void* dst_buffer, uint64_t dst_offset, const void* src, uint64_t bytes);
int smith_copy_d2h(void* ctx, void* dst, const void* src_buffer, uint64_t src_offset, uint64_t bytes);
int smith_copy_d2d(void* ctx, void* dst_buffer, uint64_t dst_offset, const void* src_buffer,
                   uint64_t src_offset, uint64_t bytes);
/* rows x width bytes between pitched device regions (no reference
 * counterpart: used to place the column ranges of mixed-type q|k|v
 * projections into one row-major output). */
int smith_copy_2d(void* ctx, void* dst, uint64_t dpitch, const void* src, uint64_t spitch, uint64_t width,
                  uint64_t rows);
int smith_fill_zero(void* ctx, void* buffer, uint64_t bytes); /* enqueued fill kernel */

/* Fusion hint, no counterpart in the reference (for host loops that run
 * GEMM after GEMM on the same rows, such as a prompt's layers): the next
 * matmul / linear call that takes the MFMA GEMM path and ends in a K-split
 * reduce with a residual or SwiGLU epilogue -- or the next prompt-row
 * smith_attention call, with gamma null -- also writes its output rows as
 * the f16 A operand of the GEMM after it (RMS-normalised with gamma when
 * gamma is non-null, with eps), and that GEMM skips its own activation prep
 * if it reads exactly those rows with the same gamma and eps.  Any other op
 * between the two must not modify those rows.  The hint, and the prepared
 * operand it leads to, are dropped by every kernel launch of any other call
 * (op entry points, smith_fill_zero, generic dispatches) and every copy into
 * device memory. */
int smith_prep_next(void* ctx, const float* gamma, float eps);

int smith_sync(void* ctx);
void smith_free(void* p); /* strings and SmithTiming returned by this library */
const char* smith_last_error(void* ctx);

/* ---- code objects (gpu_bridge.h:57-64) ---- */
/* Load a gfx950 code object (.hsaco) from disk (hipModuleLoad).  The first
 * library loaded also provides the kernels of the op-level entry points. */
void* smith_load_library(void* ctx, const char* path);
/* Compile HIP source for gfx950 with hipRTC and load it. */
void* smith_compile_source(void* ctx, const char* source, char** error_out);
void* smith_create_pipeline(void* ctx, void* library, const char* fn_name);

/* ---- encoded dispatch (gpu_bridge.h:72-99) ----
 * Buffers and inline bytes bind to argument slots by index; at dispatch the
 * slots are packed in index order into the kernel-argument block (a buffer is
 * an 8-byte pointer; inline bytes are aligned to 8 if their length is a
 * multiple of 8, else to 4).  smith_dispatch follows Metal dispatchThreads:
 * grid_* is the TOTAL thread count per dimension and the launch uses
 * ceil(grid/group) workgroups, so kernels bound-check their indices. */
SmithEncoder* smith_begin(void* ctx);
void smith_set_buffer(SmithEncoder* enc, void* buffer, uint32_t index);
void smith_set_bytes(SmithEncoder* enc, const void* data, uint32_t length, uint32_t index);
void smith_set_pipeline(SmithEncoder* enc, void* pipeline);
void smith_set_threadgroup_memory(SmithEncoder* enc, uint64_t length, uint32_t index);
void smith_dispatch(SmithEncoder* enc, uint64_t grid_x, uint64_t grid_y, uint64_t grid_z,
                    uint64_t group_x, uint64_t group_y, uint64_t group_z);
void smith_end_sync(SmithEncoder* enc);
void* smith_end_async(SmithEncoder* enc);
void smith_wait(void* token);
SmithTiming* smith_end_timed(SmithEncoder* enc);
void smith_dispatch_sync(void* ctx, void* pipeline, void** buffers, uint32_t* indices, uint32_t buffer_count,
                         const void* params, uint32_t params_length, uint32_t params_index, uint64_t grid_x,
                         uint64_t grid_y, uint64_t grid_z, uint64_t group_x, uint64_t group_y,
                         uint64_t group_z);

/* ---- op-level entry points (new: one FFI call per op) ----
 * All are enqueued on the context stream and return without waiting.
 * Buffers are device pointers.  Formats are byte-exact with the reference. */

/* quantizeQ4 (src/ops/quantize.js:14-68) on the GPU: w is f32 [K,N]
 * row-major; out receives ceil(K/32)*N*24 bytes of Q4S records. */
int smith_quantize_q4(void* ctx, const float* w, void* out, uint32_t K, uint32_t N);

/* Q8 blocks in the layout matmulQ8 consumes (shaders/matmul_q8.metal:40-52);
 * the reference has no Q8 quantizer, the rounding is ggml's q8_0 reference.
 * out receives ceil(K/32)*N*34 bytes. */
int smith_quantize_q8(void* ctx, const float* w, void* out, uint32_t K, uint32_t N);

/* matmulQ4 (src/ops/quantize.js:71-90): out[M,N] = a[M,K] . deq(wq).
 * M < 64 (or K % 32 != 0) runs the decode GEMVs on 32-row chunks, which
 * keep the reference's f32 range (a sum the f16 operands overflow, or an
 * inf / NaN activation, is redone in f32); M >= 64 with K % 32 == 0 runs
 * the f16 MFMA GEMM, which needs |a| < 65504. */
int smith_matmul_q4(void* ctx, const float* a, const void* wq, float* out, uint32_t M, uint32_t N,
                    uint32_t K, uint32_t groups);

/* smith_matmul_q4 without any allocation.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * kernels and results as smith_matmul_q4, but the split-K partials,
 * counters and activation staging live in a static 32 MiB device array per
 * GPU (held until the process ends): 64 KiB of counters, 4 MiB of
 * activation staging, the rest split-K partials.  A shape whose scratch does
 * not fit returns -1 with the sizes in smith_last_error (e.g. the M >= 256
 * prefill GEMM at K = 14336); no hipMalloc / hipFree is ever called.  Calls
 * that overlap on one GPU (two contexts or streams at once) race on the
 * array: a second host thread entering while one is enqueueing fails with an
 * error, but work of two streams overlapping on the GPU is not detected.
 * The split-K counters in the array return to zero at the end of every
 * launch that completes; a launch that faults ends the process's device
 * context anyway. */
int smith_matmul_q4_noalloc(void* ctx, const float* a, const void* wq, float* out, uint32_t M, uint32_t N,
                            uint32_t K, uint32_t groups);

/* matmulQ8 (src/ops/quantize.js:99-118): out[M,N] = a[M,K] . deq(wq). */
int smith_matmul_q8(void* ctx, const float* a, const void* wq, float* out, uint32_t M, uint32_t N,
                    uint32_t K, uint32_t groups);

/* GGUF Q4_0 weight (src/gguf.js:187-197), listed [out=N, in=K] in the file
 * (K % 32 == 0).  smith_repack_q4_0 moves the N*K/32 18-byte blocks into the
 * planar layout the GEMV reads (nib: N*K/2 bytes, d: N*K/32 f16) without
 * changing a byte; smith_matmul_q4_0 computes out[M,N] = a[M,K] . W^T, the
 * product gguf_loader.js:243-253 forms after transposing an [out,in] weight. */
int smith_repack_q4_0(void* ctx, const void* blocks, void* nib, void* d, uint32_t N, uint32_t K);
int smith_matmul_q4_0(void* ctx, const float* a, const void* nib, const void* d, float* out, uint32_t M,
                      uint32_t N, uint32_t K);

/* GGUF Q4_0 encoder (ggml q4_0 rounding, the reference decoder's interleaved
 * nibble order) for a row-major f32 [rows, cols] matrix, cols % 32 == 0.
 * Used to write synthetic GGUF files; out receives rows*cols/32*18 bytes. */
int smith_quantize_q4_0(void* ctx, const float* x, void* out, uint32_t rows, uint32_t cols);

/* ---- GGUF Llama decode path (loadGGUF(...).generate) ----
 * Weights listed [out=N, in=K] in the file.  The *_into repacks place column
 * n of a weight at column n_off + n*n_stride of a shared N_total-column
 * buffer (q|k|v concatenated; gate/up interleaved for the SwiGLU epilogue),
 * moving blocks without changing a byte (gguf_loader.js:216-273 dequantizes
 * everything to f32 instead; keeping the blocks is what makes the decode
 * HBM-bound on 4.5 bits per weight). */
int smith_repack_q4_0_into(void* ctx, const void* blocks, void* nib, void* d, uint32_t N, uint32_t K,
                           uint32_t n_off, uint32_t n_stride, uint32_t N_total);
int smith_repack_q8_0_into(void* ctx, const void* blocks, void* dst, uint32_t N, uint32_t K, uint32_t n_off,
                           uint32_t n_stride, uint32_t N_total);
/* linear (nn.js:22-25) on a repacked Q4_0 / Q8 weight with optional fusions:
 * norm_gamma != NULL: RMSNorm of each x row first (rmsnorm.metal:15-47);
 * epilogue 0: out = y; 1: out = resid + y (gguf_cache.js:159,171);
 * 2: columns are (gate, up) pairs, out[M, N/2] = silu(gate) * up
 * (swiglu.metal:12-21). */
int smith_linear_q4_0(void* ctx, const float* x, const void* nib, const void* d, float* out, uint32_t M, uint32_t N,
                      uint32_t K, const float* norm_gamma, float eps, const float* resid, uint32_t epilogue);
int smith_linear_q8(void* ctx, const float* x, const void* wq, float* out, uint32_t M, uint32_t N, uint32_t K,
                    const float* norm_gamma, float eps, const float* resid, uint32_t epilogue);
/* Q4_0 in tile-major planes (16-column tiles, each G*256 nibble bytes
 * contiguous; f16 scales at the same record index): the layout the decode
 * kernels stream.  N_total % 16 == 0.  Same placement rules as
 * smith_repack_q4_0_into. */
int smith_repack_q4_0_t_into(void* ctx, const void* blocks, void* nib, void* d, uint32_t N, uint32_t K,
                             uint32_t n_off, uint32_t n_stride, uint32_t N_total);
/* smith_linear_q4_0 on tile-major planes (N % 16 == 0). */
int smith_linear_q4_0_t(void* ctx, const float* x, const void* nib, const void* d, float* out, uint32_t M,
                        uint32_t N, uint32_t K, const float* norm_gamma, float eps, const float* resid,
                        uint32_t epilogue);
/* Single-row linear on a prepared activation ("act": the input vector in the
 * MFMA operand form plus per-8-element sums, K*4 + K/8*12 bytes) written by
 * the producing kernel.  norm != 0: RMSNorm of the input (its gamma was
 * applied when the act was written; rms comes from the act's sums of
 * squares).  Epilogues as smith_linear_q4_0; out may be NULL.  act_out !=
 * NULL: also write the act of the output vector (times gamma_out, when not
 * NULL) for the next projection; the output length must be a multiple of
 * 32.  Same results as smith_linear_q4_0_t up to f32 rounding order. */
int smith_linear_q4_0_t_act(void* ctx, const void* act_in, int norm, float eps, const void* nib, const void* d,
                            float* out, uint32_t N, uint32_t K, const float* resid, uint32_t epilogue,
                            void* act_out, const float* gamma_out);
/* rmsnormForward (ops/rmsnorm.js:19-37) over rows. */
int smith_rmsnorm(void* ctx, const float* x, const float* gamma, float* out, uint32_t rows, uint32_t cols, float eps);
/* embedding gather (autograd.js:308-334): out[r] = E[tokens[r]]; with
 * act_out (rows == 1) also the act of out times gamma_out. */
int smith_embed(void* ctx, const float* E, const int32_t* tokens, float* out, uint32_t rows, uint32_t dim,
                void* act_out, const float* gamma_out);
/* RoPE (whole-row indexing of rope.metal:18-37 as gguf_cache.js applies it)
 * + KV-cache append + GQA softmax attention for S rows at positions
 * *pos_ptr .. *pos_ptr+S-1 (gguf_cache.js:128-157, 212-231).  qkv rows are
 * [q | k | v] with stride ld; caches are [n_kv_heads, max_seq, head_dim];
 * head_dim <= 128 and a multiple of 4.  act_out (S == 1): also the act of
 * the output row for the output projection.
 * rope_cos / rope_sin hold rope_len entries each.  The position lives in
 * device memory, so its bound is checked on the device: when
 * *pos_ptr + S > max_seq or (*pos_ptr + S) * (n_heads*head_dim/2) > rope_len
 * (the whole-row RoPE of a q row would read past the table, where the
 * reference reads out of bounds, rope.metal:29-36) the kernels touch no
 * cache or table entry, and the next synchronising call (smith_sync,
 * smith_copy_d2h) returns -1 with the positions in smith_last_error. */
int smith_attention(void* ctx, const float* qkv, uint32_t ld, const int32_t* pos_ptr, uint32_t S, uint32_t n_heads,
                    uint32_t n_kv_heads, uint32_t head_dim, const float* rope_cos, const float* rope_sin,
                    uint32_t rope_len, float* kcache, float* vcache, uint32_t max_seq, float* out, void* act_out);
/* Single-row attention (S == 1, position *pos_ptr) that leaves the
 * combination of its key splits to the output projection: parts receives,
 * per head and split, (m, l, pad, pad, o[head_dim]) in 132-float records
 * (n_heads * 8 * 132 floats); caches appended as smith_attention.
 * rope_row (may be NULL): 4 + n_heads*head_dim + n_kv_heads*head_dim floats
 * that smith_argmax_embed fills with the cos / sin table entries of the next
 * position (int32 tag = that position in the first word); when the tag is
 * *pos_ptr the RoPE reads them instead of the table (one memory round trip
 * less), otherwise the table.  head_dim <= 128, % 32.  Position bound
 * (*pos_ptr + 1 against max_seq and rope_len) checked on the device as in
 * smith_attention. */
int smith_attention_parts(void* ctx, const float* qkv, const int32_t* pos_ptr, uint32_t n_heads, uint32_t n_kv_heads,
                          uint32_t head_dim, const float* rope_cos, const float* rope_sin, uint32_t rope_len,
                          const float* rope_row, float* kcache, float* vcache, uint32_t max_seq, float* parts);
/* smith_linear_q4_0_t_act whose input is smith_attention_parts' partials
 * (K = n_heads * head_dim; the splits are combined per head first). */
int smith_linear_q4_0_t_attn(void* ctx, const float* parts, const int32_t* pos_ptr, uint32_t head_dim,
                             const void* nib, const void* d, float* out, uint32_t N, uint32_t K, const float* resid,
                             uint32_t epilogue, void* act_out, const float* gamma_out);
/* Other GGUF block types on the quantized path (src/gguf.js:203-339 decode
 * them to f32 at load; here the blocks stay quantized).  A weight listed
 * [out=N, in=K] of GGML type Q4_0 (2), Q4_1 (3), Q5_0 (6), Q4_K (12) or
 * Q6_K (14) is moved into one "tile plane" buffer of
 * smith_gguf_tiles_bytes(type, N_total, K) bytes (0: shape or type not
 * supported; N % 16 == 0, K % 32 == 0, K % 256 == 0 for Q4_K / Q6_K):
 * nibbles, high bits, per-32 scales, per-256 scales, each in 16-column tiles.
 * smith_repack_gguf_tiles_into places the N rows of `blocks` at columns
 * n_off + n * n_stride of an N_total-column buffer (fused q|k|v, interleaved
 * gate/up), as smith_repack_q4_0_t_into does.
 * smith_linear_gguf_tiles: y = x . W^T for M rows with the fused RMSNorm /
 * residual / SwiGLU of smith_linear_q4_0_t (Q4_0 runs exactly that; the
 * other types run the MFMA GEMM, f16 weights, for every M).
 * smith_linear_gguf_tiles_act / _attn: the single-row act GEMVs of
 * smith_linear_q4_0_t_act / _attn on these planes (exact weights). */
uint64_t smith_gguf_tiles_bytes(uint32_t ggml_type, uint32_t N, uint32_t K);
int smith_repack_gguf_tiles_into(void* ctx, uint32_t ggml_type, const void* blocks, void* planes, uint32_t N,
                                 uint32_t K, uint32_t n_off, uint32_t n_stride, uint32_t N_total);
int smith_linear_gguf_tiles(void* ctx, uint32_t ggml_type, const float* x, const void* planes, float* out,
                            uint32_t M, uint32_t N, uint32_t K, const float* norm_gamma, float eps, const float* resid,
                            uint32_t epilogue);
int smith_linear_gguf_tiles_act(void* ctx, uint32_t ggml_type, const void* act_in, int norm, float eps,
                                const void* planes, float* out, uint32_t N, uint32_t K, const float* resid,
                                uint32_t epilogue, void* act_out, const float* gamma_out);
int smith_linear_gguf_tiles_attn(void* ctx, uint32_t ggml_type, const float* parts, const int32_t* pos_ptr,
                                 uint32_t head_dim, const void* planes, float* out, uint32_t N, uint32_t K,
                                 const float* resid, uint32_t epilogue, void* act_out, const float* gamma_out);
/* One launch for a q|k|v whose weights differ in block type: output columns
 * [0, N1) from planes1 (type1, e.g. q|k in Q4_K), [N1, N1 + N2) from planes2
 * (type2, e.g. v in Q6_K), both on the same act (optional RMSNorm scale);
 * plain stores.  smith_gguf_tiles_pair_ok tells which pairs have a kernel
 * (Q4_K+Q6_K, Q4_K+Q5_0, Q5_0+Q6_K, Q4_0+Q6_K, Q4_K+Q4_0). */
int smith_gguf_tiles_pair_ok(uint32_t type1, uint32_t type2);
int smith_linear_gguf_tiles_pair_act(void* ctx, uint32_t type1, const void* planes1, uint32_t N1, uint32_t type2,
                                     const void* planes2, uint32_t N2, const void* act_in, int norm, float eps,
                                     float* out, uint32_t K);
/* LM head on a Q6_K output.weight read as lmHead[K=dim][N=vocab] (256-element
 * blocks along vocab, dequantQ6_K src/gguf.js:309-339): the blocks are split
 * into one plane buffer of smith_lmhead_q6_k_bytes(K, N) bytes (nibbles and
 * high bits in row octets, int8 scales and f16 d; N % 256 == 0, K % 8 == 0
 * for the repack), then
 * y = rmsnorm(x, gamma) . lmHead as smith_lmhead_q4_0_nb (K % 16 == 0). */
uint64_t smith_lmhead_q6_k_bytes(uint32_t K, uint32_t N);
int smith_repack_lmhead_q6_k(void* ctx, const void* blocks, void* planes, uint32_t K, uint32_t N);
int smith_lmhead_q6_k_nb(void* ctx, const float* x, const float* norm_gamma, float eps, const void* planes, float* y,
                         uint32_t K, uint32_t N);
/* smith_lmhead_q6_k_nb followed by the greedy step in the same launch, as
 * smith_lmhead_q4_0_greedy does for the Q4_0 head (gguf_cache.js:174-184,
 * generate.js:70-76, gguf_cache.js:335-341).  Calls on one context must not
 * overlap (one device-side argmax slot). */
int smith_lmhead_q6_k_greedy(void* ctx, const float* x, const float* norm_gamma, float eps, const void* planes,
                             float* logits, uint32_t K, uint32_t N, const float* E, float* x_out, int32_t* tokens,
                             int32_t* count, int32_t* pos, void* act_out, const float* gamma_out,
                             const float* rope_cos, const float* rope_sin, uint32_t rope_len, uint32_t wq,
                             uint32_t wk, float* rope_row);
/* dequantizeTensor (src/gguf.js:343-394) on the device: numel elements of a
 * flat GGUF tensor of type F32, F16, BF16, Q4_0, Q4_1, Q5_0, Q8_0, Q4_K or
 * Q6_K to f32, bit-identical to the reference's Float32Array. */
int smith_dequantize_gguf(void* ctx, uint32_t ggml_type, const void* src, float* dst, uint64_t numel);
/* LM head on a Q4_0 output.weight read as lmHead[K=dim][N=vocab] (blocks run
 * along the vocab axis, gguf_loader.js:240-259): smith_repack_lmhead_q4_0
 * regroups the raw blocks by row octets into a nibble plane (K*N/2 bytes:
 * record (k/8, vocab block) = 8 rows x 16 nibble bytes, quarter-major) and a
 * scale plane (K*N/16 bytes: the 8 f16 scales of each record);
 * smith_lmhead_q4_0_nb computes y = x . lmHead on those planes, optional
 * fused final RMSNorm.  K % 8 == 0, K <= 8192, N % 32 == 0.
 * Replaces the f32 lm-head matmul of gguf_cache.js:174-184. */
int smith_repack_lmhead_q4_0(void* ctx, const void* blocks, void* nib, void* d, uint32_t K, uint32_t N);
int smith_lmhead_q4_0_nb(void* ctx, const float* x, const float* norm_gamma, float eps, const void* nib,
                         const void* d, float* y, uint32_t K, uint32_t N);
/* smith_lmhead_q4_0_nb followed by smith_argmax_embed's greedy step in the
 * same launch (gguf_cache.js:174-184 then generate.js:70-76 and the token
 * append of gguf_cache.js:335-341): logits are written as by
 * smith_lmhead_q4_0_nb; token = first maximum of the logits (a NaN at index 0
 * gives 0, as the reference's scan), tokens[*count] = token, x_out =
 * E[token] (may be x: it is written after every read of x), ++*count, ++*pos,
 * the act of x_out times gamma_out and the rope row as smith_argmax_embed.
 * Calls on one context must not overlap (one device-side argmax slot). */
int smith_lmhead_q4_0_greedy(void* ctx, const float* x, const float* norm_gamma, float eps, const void* nib,
                             const void* d, float* logits, uint32_t K, uint32_t N, const float* E, float* x_out,
                             int32_t* tokens, int32_t* count, int32_t* pos, void* act_out, const float* gamma_out,
                             const float* rope_cos, const float* rope_sin, uint32_t rope_len, uint32_t wq,
                             uint32_t wk, float* rope_row);
/* f32 GEMV, W [K][N] (w_is_nk = 0) or [N][K] (weight tying, 1). */
int smith_gemv_f32(void* ctx, const float* x, const float* norm_gamma, float eps, const float* W, float* y,
                   uint32_t K, uint32_t N, int w_is_nk);
/* greedy step on device: token = argmax(logits) (generate.js:70-76),
 * tokens[*count] = token, x = E[token], ++*count, ++*pos; with act_out also
 * the act of x times gamma_out.  With rope_row (may be NULL) also the rope
 * row of the new position for smith_attention_parts (q rows wq wide, k rows
 * wk wide; written only when the tables, rope_len entries each, reach it). */
int smith_argmax_embed(void* ctx, const float* logits, uint32_t N, const float* E, uint32_t dim, float* x,
                       int32_t* tokens, int32_t* count, int32_t* pos, void* act_out, const float* gamma_out,
                       const float* rope_cos, const float* rope_sin, uint32_t rope_len, uint32_t wq, uint32_t wk,
                       float* rope_row);
int smith_set_i32(void* ctx, int32_t* p, int32_t v);
/* seeded N(mean, std) f32 stream (SplitMix64 + Box-Muller), offset even. */
int smith_randn(void* ctx, float* out, uint64_t n, uint64_t seed, uint64_t offset, float stdv, float mean);

/* ---- HIP graphs: capture the context stream, replay it ----
 * Ops enqueued between begin and end are recorded, not run; their scratch
 * must already be allocated (run the same ops once before capturing).
 * Scratch that a later, bigger op replaces stays allocated until
 * smith_destroy, so a graph captured earlier stays valid. */
int smith_graph_begin(void* ctx);
void* smith_graph_end(void* ctx);
int smith_graph_launch(void* ctx, void* graph);
void smith_graph_destroy(void* graph);

/* ---- timing on the context stream (HIP events) ---- */
/* While enabled, every op-level kernel launch is bracketed by a HIP event
 * pair on the context stream.  smith_profile_read waits for the stream and
 * returns (then forgets) the summed duration and count of the recorded
 * launches whose kernel name starts with prefix (all if prefix is NULL/""). */
int smith_profile_kernels(void* ctx, int enable);
int smith_profile_read(void* ctx, const char* prefix, double* total_ms, uint64_t* count);
int smith_timer_start(void* ctx);
/* Waits for the stream; returns milliseconds since smith_timer_start, <0 on error. */
double smith_timer_stop(void* ctx);

#ifdef __cplusplus
}
#endif
#endif
