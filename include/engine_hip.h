/*
 * engine_hip.h -- C-ABI of the MI355X (gfx950) matrix-multiply engine.
 *
 * This is the drop-in boundary. It is plain C: no HIP, torch or C++ types
 * cross it. Device pointers are `void*`/typed pointers to device memory,
 * streams and events are opaque handles (a HIP stream handle may be passed
 * where an `eng_stream` is expected; NULL is the legacy default stream),
 * dimensions are signed 64-bit, and every function returns a status code:
 *
 *   ENG_OK (0)                 success
 *   ENG_INVALID_ARGUMENT (1)   a precondition failed; nothing was launched
 *   ENG_DEVICE_ERROR (2)       the HIP runtime reported an error
 *
 * After a non-zero status, eng_last_error() returns the message of the
 * failure on the calling thread, formatted like the reference's EngineError:
 *   "[engine] <file>:<line>\n  check failed: <expr>\n  <message>"
 * and containing the same substrings the reference's contract tests match
 * ("null", "non-negative", "negative", "eps").
 *
 * The C++17 launch API of the reference (namespace engine::cuda, header
 * include/engine/kernels.hpp) is restated on top of this ABI by the headers
 * under include/engine/ in this repository.
 *
 * Layout convention (reference include/engine/cpu_ref.hpp:14-17): all 2-D
 * data is row-major and contiguous. GEMV/RMSNorm+linear weights are stored
 * [K x N] and out = x . W (reference include/engine/kernels.hpp:83-99).
 */
#ifndef ENGINE_HIP_H
#define ENGINE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ENG_OK 0
#define ENG_INVALID_ARGUMENT 1
#define ENG_DEVICE_ERROR 2

/* IEEE-754 binary16 bit pattern (the reference's engine::half). */
typedef uint16_t eng_half;
/* Opaque stream / event handles (hipStream_t / hipEvent_t underneath). */
typedef void* eng_stream;
typedef void* eng_event;
/* Opaque pooled-allocator handle. */
typedef struct eng_pool_s* eng_pool;

/* Device kinds, numbered like the reference's engine::Device
 * (include/engine/tensor.hpp:50-53): 0 = host, 1 = the GPU. */
#define ENG_DEVICE_CPU 0
#define ENG_DEVICE_GPU 1

/* Stream / event flags (values of hipStreamNonBlocking / hipEventDisableTiming). */
#define ENG_STREAM_DEFAULT 0u
#define ENG_STREAM_NON_BLOCKING 1u
#define ENG_EVENT_DEFAULT 0u
#define ENG_EVENT_DISABLE_TIMING 2u

/* Message of the last failed call on this thread ("" if none). */
const char* eng_last_error(void);
/* Library build string: "engine_hip <version> gfx950 <build flags> git <source revision>". */
const char* eng_build_info(void);

/* ------------------------------------------------------------------------
 * Device queries. Replace engine::cuda_device_count / cuda_device_summary /
 * cuda_peak_bandwidth_gbs / cuda_driver_version / cuda_clock_rate_khz /
 * cuda_live_sm_clock_mhz / cuda_live_mem_clock_mhz
 * (reference include/engine/cuda_device.hpp:20-48, src/cuda_device.cpp:51-222).
 * Like the reference, the count answers 0 (not an error) when no device or
 * driver is present.
 * ---------------------------------------------------------------------- */
int eng_device_count(int* count);
int eng_device_summary(char* buf, size_t len);
/* Theoretical peak HBM bandwidth from the device's memory clock and bus
 * width (clock x bus bytes x 2), in GB/s. */
int eng_peak_bandwidth_gbs(double* gbs);
int eng_driver_version(char* buf, size_t len);
int eng_clock_rate_khz(int* khz);
/* Live clocks in MHz, read on each call from the amdgpu driver's sysfs node
 * of the device's PCI function: the current level of pp_dpm_sclk /
 * pp_dpm_mclk, else the hwmon freq1_input / freq2_input. Without either, the
 * engine clock falls back to the nominal clock and the memory clock reports 0,
 * as the reference does without NVML (src/cuda_device.cpp:196-222).
 * eng_live_clock_source names the files read ("unavailable" for a fallback). */
int eng_live_sm_clock_mhz(int* mhz);
int eng_live_mem_clock_mhz(int* mhz);
int eng_live_clock_source(char* buf, size_t len);
/* Architecture the device reports (e.g. "gfx950:sramecc+:xnack-"). */
int eng_device_arch(char* buf, size_t len);
int eng_device_cu_count(int* cus);

/* ------------------------------------------------------------------------
 * Memory. Replace the cudaMalloc / cudaFree / cudaMemcpy / cudaMemset calls
 * behind engine::DeviceBuffer<T> (reference include/engine/device_buffer.hpp:
 * 33-92) and Storage (src/tensor.cpp:56-95).
 * ---------------------------------------------------------------------- */
int eng_malloc(void** ptr, size_t bytes);
int eng_free(void* ptr);
/* The blocking calls (eng_memcpy_h2d / _d2h / _d2d, eng_memset) have finished
 * on the device when they return, so work queued afterwards on any stream,
 * non-blocking ones included, sees their bytes. */
int eng_memcpy_h2d(void* dst, const void* src, size_t bytes);
int eng_memcpy_d2h(void* dst, const void* src, size_t bytes);
int eng_memcpy_d2d(void* dst, const void* src, size_t bytes);
int eng_memcpy_h2d_async(void* dst, const void* src, size_t bytes, eng_stream stream);
int eng_memcpy_d2h_async(void* dst, const void* src, size_t bytes, eng_stream stream);
int eng_memset(void* ptr, int value, size_t bytes);
/* The low byte of `value` into `bytes` bytes, ordered on `stream`. A fill
 * kernel (not hipMemsetAsync), so it may be captured into a HIP graph. */
int eng_memset_async(void* ptr, int value, size_t bytes, eng_stream stream);
int eng_device_sync(void);
/* hipGetLastError(), cleared; ENG_DEVICE_ERROR with its text if set. */
int eng_check_last_launch(void);

/* ------------------------------------------------------------------------
 * Streams and events. Replace engine::CudaStream / CudaEvent
 * (reference include/engine/cuda_stream.hpp:21-124, src/cuda_stream.cpp:11-38).
 * Streams are created at the default priority. eng_stream_destroy waits for
 * the stream's work and releases the stream's scratch arena (the device
 * memory the split-K GEMV, split-KV attention, rmsnorm_linear at M > 1 and the
 * FFN launchers reuse on that stream; it grows to the largest request).
 * ---------------------------------------------------------------------- */
int eng_stream_create(eng_stream* stream, unsigned int flags);
int eng_stream_destroy(eng_stream stream);
int eng_stream_sync(eng_stream stream);
int eng_stream_wait_event(eng_stream stream, eng_event event, unsigned int flags);
/* Holds `stream` for `microseconds` of GPU time (at most 1,000,000): one
 * one-wave kernel that sleeps until the device's constant-rate clock has
 * advanced that far, then exits. A timing harness issues it before a window
 * of launches so that every launch of the window is queued before the first
 * one starts and the window measures the GPU's back-to-back rate, not the
 * host's issue rate (no reference counterpart; the reference's harness times
 * launches as the host issues them, bench/bench_harness.hpp:205-348). */
int eng_stream_delay(eng_stream stream, unsigned int microseconds);
int eng_event_create(eng_event* event, unsigned int flags);
int eng_event_destroy(eng_event event);
int eng_event_record(eng_event event, eng_stream stream);
/* *done = 1 when complete, 0 when still pending. */
int eng_event_query(eng_event event, int* done);
int eng_event_sync(eng_event event);
int eng_event_elapsed_ms(float* ms, eng_event start, eng_event end);

/* ------------------------------------------------------------------------
 * HIP graph capture of a stream. No counterpart in the reference: for decode
 * loops that issue the same launches every token (capture once, replay per
 * token). eng_graph_capture_begin starts recording the work issued on
 * `stream` (a stream from eng_stream_create, not the null stream) without
 * running it; eng_graph_capture_end stops, instantiates and returns the graph;
 * eng_graph_launch replays it on any stream. Every launcher here is
 * capture-safe once it has run eagerly on that stream at least once with
 * shapes at least as large (the stream's scratch arena is sized outside the
 * capture -- a call that would have to grow it during capture fails with a
 * message saying so; zero fills are kernels, not memsets). A failed capture
 * returns an error and leaves no graph; the stream is no longer capturing
 * either way.
 * Scratch: at capture end the call waits for the capture stream's earlier
 * (eager) work, then the graph takes over the blocks of the capture stream's
 * scratch arenas that launches captured in it leased, and the stream continues
 * on fresh blocks of the same sizes. A replay therefore shares no scratch with
 * eager calls on the capture stream or with any other graph, may run on any
 * stream, and stays valid after the capture stream is destroyed. Replays of
 * one graph share its blocks: they must not overlap (issue them on one
 * stream, or order them with events). eng_graph_destroy waits for the device
 * before freeing the graph's blocks.
 * ---------------------------------------------------------------------- */
typedef void* eng_graph;
int eng_graph_capture_begin(eng_stream stream);
int eng_graph_capture_end(eng_stream stream, eng_graph* graph);
int eng_graph_launch(eng_graph graph, eng_stream stream);
int eng_graph_destroy(eng_graph graph);

/* ------------------------------------------------------------------------
 * Pooled allocator. Replaces engine::PoolAllocator / pool_allocator(Device) /
 * AllocStats (reference include/engine/pool_allocator.hpp:27-148,
 * include/engine/allocator.hpp:34-63, src/pool_allocator.cpp:38-271):
 * power-of-two buckets of at least 256 B, 256-B alignment, slabs carved
 * most-recent-first, slab size doubling from the initial size and capped at
 * 64 MiB, stream-ordered reuse of GPU blocks through a per-block event,
 * mutex-guarded, exact statistics.
 * ---------------------------------------------------------------------- */
typedef struct eng_alloc_stats {
  uint64_t bytes_in_use;
  uint64_t bytes_reserved;
  uint64_t peak_bytes_in_use;
  uint64_t num_allocs;
  uint64_t num_driver_allocs;
} eng_alloc_stats;

int eng_pool_create(eng_pool* pool, int device, size_t initial_slab_bytes);
int eng_pool_destroy(eng_pool pool);
/* The process-wide pool of a device kind (created on first use). */
int eng_pool_default(eng_pool* pool, int device);
/* bytes == 0 yields *ptr == NULL and ENG_OK, like the reference. */
int eng_pool_allocate(eng_pool pool, size_t bytes, void** ptr);
/* Host pools: immediate. GPU pools: reuse deferred until the work queued on
 * `stream` so far completes (an event is recorded on `stream`). */
int eng_pool_deallocate(eng_pool pool, void* ptr, eng_stream stream);
int eng_pool_stats(eng_pool pool, eng_alloc_stats* stats);
int eng_pool_reset(eng_pool pool);
/* Passthrough allocator of a device kind (reference src/allocator.cpp:42-118). */
int eng_passthrough_allocate(int device, size_t bytes, void** ptr);
int eng_passthrough_deallocate(int device, void* ptr);
int eng_passthrough_stats(int device, eng_alloc_stats* stats);

/* ------------------------------------------------------------------------
 * Host fp16 conversions (IEEE-754 round-to-nearest-even; replaces the
 * host half_to_float / float_to_half of reference include/engine/half.hpp:
 * 27-105, whose non-CUDA float->half truncates).
 * ---------------------------------------------------------------------- */
int eng_f32_to_f16_host(const float* in, eng_half* out, size_t n);
int eng_f16_to_f32_host(const eng_half* in, float* out, size_t n);

/* ------------------------------------------------------------------------
 * Kernels. All pointers are DEVICE pointers; launches are asynchronous on
 * `stream`. Preconditions, messages and zero-size behaviour follow the
 * reference launchers exactly:
 *   - null pointer           -> ENG_INVALID_ARGUMENT, "... is null" / "null device pointer"
 *   - negative dimension     -> ENG_INVALID_ARGUMENT, "... must be non-negative" / "negative dimension"
 *   - GEMV/GEMM with K == 0  -> output zero-filled on `stream`
 *   - N == 0 (GEMV), M or N == 0 (GEMM) -> no-op
 *   - rmsnorm_linear with any dimension 0 -> no-op (nothing written)
 * ---------------------------------------------------------------------- */

/* C[M x N] = A[M x K] . B[K x N], fp32 accumulate, on FP32 MFMA.
 * Replaces engine::cuda::matmul_register_tiled
 * (reference include/engine/kernels.hpp:77-81, kernels/matmul_register_tiled.cu:176-199). */
int eng_matmul_f32(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                   eng_stream stream);

/* out[N] = x[K] . A[K x N], fp32. Replaces engine::cuda::gemv
 * (reference include/engine/kernels.hpp:83-86, kernels/gemv.cu:114-147). */
int eng_gemv_f32(const float* A, const float* x, float* out, int64_t N, int64_t K,
                 eng_stream stream);

/* out[N] = x[K] . A[K x N] with half A, x and out, fp32 accumulate, out
 * rounded to nearest even. Replaces engine::cuda::gemv_fp16
 * (reference include/engine/kernels.hpp:118-121, kernels/gemv_fp16.cu:117-149). */
int eng_gemv_f16(const eng_half* A, const eng_half* x, eng_half* out, int64_t N, int64_t K,
                 eng_stream stream);

/* out[N] = x[K] . A[K x N] with half A and fp32 x / out, fp32 accumulate.
 * Additive overload of engine::cuda::gemv_fp16 for fp16-weight decode with
 * fp32 activations (no reference counterpart; same contract as gemv_fp16). */
int eng_gemv_f16w(const eng_half* A, const float* x, float* out, int64_t N, int64_t K,
                  eng_stream stream);

/* out[r][c] = in[r][c] / sqrt(mean(in[r][:]^2) + eps) * weight[c]; weight may
 * be NULL (no gain). Replaces engine::cuda::rmsnorm
 * (reference include/engine/kernels.hpp:61-63, kernels/rmsnorm.cu:171-192). */
int eng_rmsnorm_f32(const float* in, const float* weight, float* out, int64_t rows,
                    int64_t cols, float eps, eng_stream stream);

/* out[M x N] = RMSNorm(in[M x K], rms_weight, eps) . W[K x N]; rms_weight may be
 * NULL. One fused kernel: the sum of squares is reduced inside the GEMV/GEMM.
 * Replaces engine::cuda::rmsnorm_linear
 * (reference include/engine/kernels.hpp:92-99, kernels/rmsnorm_linear.cu:173-201). */
int eng_rmsnorm_linear_f32(const float* in, const float* rms_weight, const float* W, float* out,
                           int64_t M, int64_t N, int64_t K, float eps, eng_stream stream);

/* As eng_rmsnorm_linear_f32 with an fp16 weight matrix W[K x N] (fp32 in / out).
 * Additive overload (no reference counterpart; same contract). */
int eng_rmsnorm_linear_f16w(const float* in, const float* rms_weight, const eng_half* W,
                            float* out, int64_t M, int64_t N, int64_t K, float eps,
                            eng_stream stream);

/* eng_rmsnorm_linear_f16w for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): no counterpart in the reference. Same arguments, kernels and
 * bits as eng_rmsnorm_linear_f16w, for M <= 16 rows (decode and small
 * batches); the split-K partial sums live in a static device buffer of
 * 8 MiB + 64 KiB per GPU, held until the process ends, instead of the stream's
 * scratch arena. Nothing is allocated. Fails with a message (status 1) for
 * M > 16 or a shape whose partial sums would exceed the buffer. Every call on
 * a GPU shares that GPU's buffer: calls that overlap on one GPU (different
 * streams or host threads without ordering) race, so order them. */
int eng_rmsnorm_linear_f16w_noalloc(const float* in, const float* rms_weight, const eng_half* W,
                                    float* out, int64_t M, int64_t N, int64_t K, float eps,
                                    eng_stream stream);

/* Output-major weights (no reference counterpart; additive). W is row-major
 * [N x K] -- one contiguous row of K weights per output, the layout of the
 * decode configurations "y = W.x, W [out x in]" -- and
 *   y[N] = W[N x K] . x[K]                                 (eng_gemv_*_nk)
 *   out[M x N] = RMSNorm(in[M x K], rms_weight, eps) . W^T  (eng_rmsnorm_linear_*_nk)
 * Same preconditions, messages and zero-size rules as the reference-layout
 * functions above (K == 0: the GEMVs zero-fill, rmsnorm_linear writes nothing).
 * Each output row is one contiguous stream, so M == 1 needs no split-K
 * reduction; M > 1 runs the FP32 MFMA GEMM with B read as B^T. */
int eng_gemv_f16w_nk(const eng_half* W, const float* x, float* y, int64_t N, int64_t K,
                     eng_stream stream);
int eng_gemv_f32_nk(const float* W, const float* x, float* y, int64_t N, int64_t K,
                    eng_stream stream);
int eng_rmsnorm_linear_f16w_nk(const float* in, const float* rms_weight, const eng_half* W,
                               float* out, int64_t M, int64_t N, int64_t K, float eps,
                               eng_stream stream);
int eng_rmsnorm_linear_f32_nk(const float* in, const float* rms_weight, const float* W,
                              float* out, int64_t M, int64_t N, int64_t K, float eps,
                              eng_stream stream);

/* Replaces engine::cuda::rmsnorm_linear_fused_direct
 * (reference include/engine/kernels.hpp:101-104, kernels/rmsnorm_linear.cu:143-171),
 * the benchmarking entry that forces the fused kernel for every M. Here every
 * M is served by fused kernels already, so it runs the same code as
 * eng_rmsnorm_linear_f32. */
int eng_rmsnorm_linear_fused_direct_f32(const float* in, const float* rms_weight,
                                        const float* W, float* out, int64_t M, int64_t N,
                                        int64_t K, float eps, eng_stream stream);

/* ------------------------------------------------------------------------
 * The ops either side of the linear layers (SwiGLU FFN, residual stream).
 * ---------------------------------------------------------------------- */

/* out[i] = a[i] + b[i], bit-exact fp32 addition. n < 0 -> "n must be
 * non-negative"; n == 0 returns before the pointer check; null -> "null device
 * pointer". Replaces engine::cuda::vector_add
 * (reference include/engine/kernels.hpp:47-50, kernels/vector_add.cu:119-149). */
int eng_vector_add_f32(const float* a, const float* b, float* out, int64_t n, eng_stream stream);

/* sum_out = x + residual (bit-exact); norm_out = sum_out / sqrt(mean(sum_out^2)
 * + eps) * weight, per row of [rows x cols]; weight may be NULL, the other
 * pointers may not ("null device pointer"); "negative dimension"; "eps must be
 * non-negative"; rows or cols == 0 writes nothing. Replaces
 * engine::cuda::residual_rmsnorm (reference include/engine/kernels.hpp:106-112,
 * kernels/residual_rmsnorm.cu:124-150). */
int eng_residual_rmsnorm_f32(const float* x, const float* residual, const float* weight,
                             float* norm_out, float* sum_out, int64_t rows, int64_t cols,
                             float eps, eng_stream stream);

/* out[i] = SiLU(gate[i]) * up[i], SiLU(g) = g / (1 + exp(-g)), fp32 (and half
 * in / out with fp32 arithmetic, rounded to nearest even). "gate is null" /
 * "up is null" / "out is null"; "n must be non-negative"; n == 0 is a no-op.
 * Replace engine::cuda::swiglu / swiglu_fp16
 * (reference include/engine/kernels.hpp:138-142, kernels/swiglu.cu:155-227). */
int eng_swiglu_f32(const float* gate, const float* up, float* out, int64_t n, eng_stream stream);
int eng_swiglu_f16(const eng_half* gate, const eng_half* up, eng_half* out, int64_t n,
                   eng_stream stream);

/* act[M x N] = SiLU(xn . Wg^T) * (xn . Wu^T), xn = RMSNorm(in[M x K], rms_weight,
 * eps), with output-major W_gate, W_up [N x K]: the gate / up half of a SwiGLU
 * FFN in one call (no reference counterpart: the reference composes rmsnorm,
 * two GEMV / GEMMs and swiglu, tests/test_kernels.cu:2867-2898). Decode
 * (M == 1) is a single fused launch; other shapes use scratch for gate
 * and up. rms_weight may be NULL. Messages: "negative dimension", "null device
 * pointer", "eps must be non-negative"; any zero dimension writes nothing. */
int eng_rmsnorm_linear_swiglu_f16w_nk(const float* in, const float* rms_weight,
                                      const eng_half* W_gate, const eng_half* W_up, float* act,
                                      int64_t M, int64_t N, int64_t K, float eps,
                                      eng_stream stream);
int eng_rmsnorm_linear_swiglu_f32_nk(const float* in, const float* rms_weight,
                                     const float* W_gate, const float* W_up, float* act,
                                     int64_t M, int64_t N, int64_t K, float eps,
                                     eng_stream stream);

/* The same with reference-layout W_gate, W_up [K x N] (the layout of
 * rmsnorm_linear, include/engine/kernels.hpp:92-99; no reference counterpart:
 * the reference composes two rmsnorm_linear calls and swiglu,
 * tests/test_kernels.cu:2867-2898). Decode (up to 16 rows, N a multiple of 8
 * fp16 / 4 fp32 elements, 16-byte aligned weights) is, per pass of up to 4
 * rows, one split-K launch over both matrices and one reduce launch with the
 * SwiGLU epilogue; its result equals that composition bit for bit. Same
 * messages as the _nk form. */
int eng_rmsnorm_linear_swiglu_f16w(const float* in, const float* rms_weight,
                                   const eng_half* W_gate, const eng_half* W_up, float* act,
                                   int64_t M, int64_t N, int64_t K, float eps,
                                   eng_stream stream);
int eng_rmsnorm_linear_swiglu_f32(const float* in, const float* rms_weight,
                                  const float* W_gate, const float* W_up, float* act, int64_t M,
                                  int64_t N, int64_t K, float eps, eng_stream stream);

/* ------------------------------------------------------------------------
 * Decode attention over an fp16 KV cache, and its bridge kernels.
 * ---------------------------------------------------------------------- */

/* Single-token decode attention with split-KV FlashDecoding: for each query
 * head h, out[h] = softmax(scale * K_g . q[h]) . V_g over keys 0..kv_len-1 of
 * KV head g = h / (n_heads / n_kv_heads). q / out [n_heads, head_dim] half;
 * K / V head-major, key j of KV head g at g * kv_head_stride + j * head_dim.
 * split_kv = 0 picks the split count; the query heads of a GQA group share
 * each K / V load. Messages (order as the reference): "q is null", "k is
 * null", "v is null", "out is null", "kv_len must be non-negative", "n_heads
 * must be positive", "n_kv_heads must be positive", "n_heads must be divisible
 * by n_kv_heads", "head_dim must be 64 or 128", "scale must be finite",
 * "split_kv must be non-negative", "kv_head_stride < kv_len * head_dim";
 * kv_len == 0 zero-fills out. Replaces engine::cuda::attention_decode
 * (reference include/engine/kernels.hpp:190-194, kernels/attention_decode.cu:
 * 632-715); the _with_mode form replaces detail::attention_decode_with_mode
 * (kernels.hpp:169-174), share_gqa_kv = 0 giving one query head per workgroup. */
int eng_attention_decode_f16(const eng_half* q, const eng_half* k, const eng_half* v,
                             eng_half* out, int64_t kv_len, int64_t n_heads, int64_t n_kv_heads,
                             int64_t head_dim, int64_t kv_head_stride, float scale, int split_kv,
                             eng_stream stream);
int eng_attention_decode_with_mode_f16(const eng_half* q, const eng_half* k, const eng_half* v,
                                       eng_half* out, int64_t kv_len, int64_t n_heads,
                                       int64_t n_kv_heads, int64_t head_dim,
                                       int64_t kv_head_stride, float scale, int split_kv,
                                       int share_gqa_kv, eng_stream stream);

/* Elementwise fp32 <-> fp16 (round to nearest even); n < 0 -> "n must be
 * non-negative", n == 0 returns before the pointer checks. Replace
 * engine::cuda::detail::cast_f32_to_f16 / cast_f16_to_f32
 * (reference include/engine/kernels.hpp:176-180, kernels/attention_bridge.cu:64-84). */
int eng_cast_f32_to_f16(const float* in, eng_half* out, int64_t n, eng_stream stream);
int eng_cast_f16_to_f32(const eng_half* in, float* out, int64_t n, eng_stream stream);

/* Scatter token-major k_new / v_new [s_new, n_kv_heads, head_dim] into
 * head-major caches [n_kv_heads, kv_max_seq_len, head_dim] at positions
 * pos_offset .. pos_offset + s_new - 1. Replaces engine::cuda::detail::kv_cache_write
 * (reference include/engine/kernels.hpp:182-188, kernels/attention_bridge.cu:86-110). */
int eng_kv_cache_write_f16(const eng_half* k_new, const eng_half* v_new, eng_half* k_cache,
                           eng_half* v_cache, int64_t s_new, int64_t n_kv_heads, int64_t head_dim,
                           int64_t pos_offset, int64_t kv_max_seq_len, eng_stream stream);

/* Weight layout conversion: dst [cols x rows] = src [rows x cols] transposed,
 * bit patterns copied unchanged. Converts reference-layout weights A [K x N]
 * (out = x . A, reference include/engine/kernels.hpp:83-99) once, at load
 * time, into the output-major W [N x K] that eng_gemv_f16w_nk /
 * eng_rmsnorm_linear_f16w_nk (and the _f32 forms) stream fastest. No
 * reference counterpart (the reference has one weight layout). Messages:
 * "negative dimension", "null device pointer", "src and dst overlap"; a zero
 * dimension is a no-op. */
int eng_transpose_f16(const eng_half* src, eng_half* dst, int64_t rows, int64_t cols,
                      eng_stream stream);
int eng_transpose_f32(const float* src, float* dst, int64_t rows, int64_t cols,
                      eng_stream stream);

/* ------------------------------------------------------------------------
 * ENGREF01 tensor files and device weight slabs.
 *
 * The container is the reference's golden format (tools/gen_reference.py:
 * 56-83, tests/golden.hpp:21-33): "ENGREF01", int32 count, then per tensor
 * int32 name length, name, int32 dtype, int32 ndim, int64 dims, int64 byte
 * count, data. The reference reader (tests/golden.cpp:104-209, which these
 * functions replace) accepts dtype 0 only; here 1 stores IEEE binary16
 * weights at native size and 2 float64. A file is memory-mapped and checked
 * as the reference checks it (messages: "bad magic", "implausible tensor
 * count", "implausible name length", "truncated tensor name", "has dtype",
 * "implausible ndim", "negative dimension", "header says ... bytes but its
 * shape implies", "truncated data", "duplicate tensor name", "unexpected
 * trailing bytes", "unexpected end of file while reading"); a missing
 * tensor name reports the names present ("not found. Available:", as
 * tests/golden.cpp:197-205). The slab is the on-disk-to-HBM step of the
 * reference's planned mmap weight loader (README.md:247): every tensor at a
 * 256-byte aligned offset, in file order, in one device allocation.
 * ---------------------------------------------------------------------- */

#define ENG_ENGREF_F32 0
#define ENG_ENGREF_F16 1
#define ENG_ENGREF_F64 2

typedef struct eng_engref_s* eng_engref;

/* Maps and validates `path`; *file is NULL on failure. A handle is
 * read-only after open and may be shared by threads. */
int eng_engref_open(const char* path, eng_engref* file);
/* Unmaps the file; pointers returned for it become invalid. NULL is a no-op. */
int eng_engref_close(eng_engref file);
int eng_engref_count(eng_engref file, int32_t* count);
/* Index of the tensor called `name` (unknown name: ENG_INVALID_ARGUMENT). */
int eng_engref_find(eng_engref file, const char* name, int32_t* index);
/* Tensor `index` (0 .. count-1, file order). Any output pointer may be NULL.
 * name (NUL-terminated), dims[ndim] and host_data (the mapped bytes,
 * little-endian, not necessarily aligned) live until eng_engref_close;
 * slab_offset is the tensor's byte offset in the slab. */
int eng_engref_tensor(eng_engref file, int32_t index, const char** name, int32_t* dtype,
                      int32_t* ndim, const int64_t** dims, int64_t* nbytes,
                      const void** host_data, int64_t* slab_offset);
/* Bytes of device memory the slab needs (a multiple of 256). */
int eng_engref_slab_bytes(eng_engref file, int64_t* bytes);
/* Copies every tensor into the caller's device allocation `slab` (256-byte
 * aligned, `capacity` >= eng_engref_slab_bytes) through pinned staging
 * buffers on `stream`; returns when the copies are complete. Padding bytes
 * between tensors are left as they were. Messages: "capacity must be
 * non-negative", "slab capacity ... bytes needed", "slab is null", "slab must
 * be 256-byte aligned". */
int eng_engref_upload(eng_engref file, void* slab, int64_t capacity, eng_stream stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* ENGINE_HIP_H */
