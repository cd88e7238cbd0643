/*
 * axon_hip — the C ABI of the MI355X (gfx950) kernel table for trickymind1324/axon-infer.
 *
 * Every pointer argument named after a tensor is a DEVICE pointer (memory from
 * axon_hip_malloc, or any HIP device allocation). Sizes are element counts unless the name
 * says bytes. Every function returns 0 on success or a negative status (AXON_HIP_E_*); the
 * message of the last failure on the calling thread is axon_hip_last_error(). Nothing here
 * throws, allocates host memory the caller must free, or falls back to the CPU: a host without
 * a usable gfx950 device gets AXON_HIP_E_NO_DEVICE from axon_hip_init.
 *
 * Kernel entries are asynchronous on the library's stream (one non-blocking stream per
 * process, default priority) and execute in call order; axon_hip_synchronize waits for them.
 *
 * The first block mirrors the reference's KernelTable one for one
 * (src/kernels/kernels.h:33-128): same names, same argument order and meaning, same layouts
 * (weights [n_out][n_in] in GGUF block layout, no transposition). The second block holds the
 * coarse entries its device-resident forward pass uses (fused norm + quantize, rope + bias +
 * KV write, SiLU + quantize, fused multi-weight matvec, ragged attention); each names the
 * reference code it replaces.
 */
#ifndef AXON_HIP_H
#define AXON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AXON_HIP_OK 0
#define AXON_HIP_E_INVALID (-1)
#define AXON_HIP_E_UNSUPPORTED (-2)
#define AXON_HIP_E_NO_DEVICE (-3)
#define AXON_HIP_E_HIP (-4)
#define AXON_HIP_E_OOM (-5)

/* ggml tensor type ids accepted by the typed entries (src/core/dtype.h:17-49). */
#define AXON_HIP_F32 0
#define AXON_HIP_F16 1
#define AXON_HIP_Q4_0 2
#define AXON_HIP_Q4_1 3
#define AXON_HIP_Q8_0 8
#define AXON_HIP_Q6_K 14
#define AXON_HIP_BF16 30

/* ---- Lifecycle: device detection, memory, stream, timing, graphs --------------------------
 * Stands where src/kernels/kernels.cpp:79-103 (select) checks the CPU: a gfx950 device must be
 * present, or AXON_HIP_E_NO_DEVICE. */
int axon_hip_device_count(int* count);
int axon_hip_init(int device);
/* Name of the device's ISA ("gfx950") into buf. */
int axon_hip_device_arch(char* buf, size_t len);
const char* axon_hip_last_error(void);
int axon_hip_malloc(void** ptr, size_t bytes);
int axon_hip_free(void* ptr);
/* Page-locked host memory for fast transfers. */
int axon_hip_host_malloc(void** ptr, size_t bytes);
int axon_hip_host_free(void* ptr);
int axon_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int axon_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);
int axon_hip_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* Asynchronous host-to-device copy on the library stream (src must stay valid until it ran). */
int axon_hip_memcpy_h2d_async(void* dst, const void* src, size_t bytes);
int axon_hip_memset(void* dst, int value, size_t bytes);
int axon_hip_synchronize(void);
int axon_hip_event_create(void** event);
/* Allocations this library's host code has made since it was loaded: *host_new counts its own
 * operator new calls, *device its device and pinned-host allocations and events
 * (axon_hip_malloc, axon_hip_host_malloc, axon_hip_event_create). No counterpart entry in the
 * reference, whose tests count a whole test binary's operator new calls
 * (tests/unit/alloc_counter.cpp:33-46): here the HIP runtime's own allocations are not this
 * library's, so each library counts its own. */
void axon_hip_allocation_counts(size_t* host_new, size_t* device);
int axon_hip_event_record(void* event);
int axon_hip_event_elapsed_ms(void* start, void* stop, float* ms);
int axon_hip_event_destroy(void* event);
/* Measurement only: the next matmul kernel launched on this thread records its own start and end
 * on these events (hipExtLaunchKernel), so their elapsed time is the kernel's duration as a
 * profiler reports it. Both NULL disarms. */
int axon_hip_probe_next_launch(void* start, void* stop);
/* Captures the entries called between begin and end into a replayable graph. */
int axon_hip_graph_begin(void);
int axon_hip_graph_end(void** graph);
int axon_hip_graph_launch(void* graph);
int axon_hip_graph_destroy(void* graph);

/* ---- The KernelTable entries (src/kernels/kernels.h:33-128) ------------------------------ */

/* kernels.h:35-39 */
int axon_hip_matmul_f32(const float* w, const float* x, float* y, size_t n_out, size_t n_in);
int axon_hip_matmul_f16(const uint16_t* w, const float* x, float* y, size_t n_out, size_t n_in);
int axon_hip_matmul_bf16(const uint16_t* w, const float* x, float* y, size_t n_out, size_t n_in);
/* kernels.h:40-47 */
int axon_hip_matmul_f32_rows(const float* w, const float* x, float* y, size_t n_rows, size_t n_out,
                             size_t n_in, size_t y_stride);
int axon_hip_matmul_f16_rows(const uint16_t* w, const float* x, float* y, size_t n_rows, size_t n_out,
                             size_t n_in, size_t y_stride);
int axon_hip_matmul_bf16_rows(const uint16_t* w, const float* x, float* y, size_t n_rows, size_t n_out,
                              size_t n_in, size_t y_stride);
/* kernels.h:49-50 */
int axon_hip_rmsnorm(const float* x, const float* weight, float* y, size_t n, float eps);
/* kernels.h:51-52 with RopeParams (kernels.h:25-31) spelled out; style 0 Normal, 1 NeoX;
 * freq_factors is a device pointer or NULL. */
int axon_hip_rope(float* x, size_t n_heads, size_t pos, size_t head_dim, size_t rotary_dim, float theta,
                  int style, const float* freq_factors);
/* kernels.h:53-54 */
int axon_hip_softmax(float* x, size_t n);
/* kernels.h:55-56 */
int axon_hip_silu_mul(const float* gate, const float* up, float* out, size_t n);
/* kernels.h:57-59 */
int axon_hip_embedding_row(int type, const void* table, size_t n, int64_t index, float* out);
/* kernels.h:60-66. scores: the reference's per-call scratch of n_q * (n_past + n_q) floats
 * (kernels.h:67-75), for attention and each of the entries below. This table keeps scores in LDS
 * and only uses the pointer for contexts too long for LDS; it then runs the call's heads one
 * after another, each within that scratch. */
int axon_hip_attention(const float* q, const float* k, const float* v, float* out, float* scores, size_t seq,
                       size_t n_head, size_t n_head_kv, size_t head_dim, float scale);
/* kernels.h:67-75 */
int axon_hip_attention_kv(const float* q, const float* k_cache, const float* v_cache, float* out, float* scores,
                          size_t n_q, size_t n_past, size_t n_head, size_t n_head_kv, size_t head_dim, float scale);
/* kernels.h:76-81 */
int axon_hip_attention_kv_heads(const float* q, const float* k_cache, const float* v_cache, float* out,
                                float* scores, size_t n_q, size_t n_past, size_t n_head, size_t n_head_kv,
                                size_t head_dim, float scale, size_t head_begin, size_t head_end);
/* kernels.h:82-87 */
int axon_hip_attention_kv_heads_f16(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                                    float* scores, size_t n_q, size_t n_past, size_t n_head, size_t n_head_kv,
                                    size_t head_dim, float scale, size_t head_begin, size_t head_end);
/* kernels.h:89-94. Blocks are the GGUF structs: Q8_0 34 bytes, Q4_0 18, Q4_1 20, Q6_K 210. */
int axon_hip_matmul_q8_0(const void* w, const float* x, float* y, size_t n_out, size_t n_in);
int axon_hip_matmul_q4_0(const void* w, const float* x, float* y, size_t n_out, size_t n_in);
/* kernels.h:95-101 */
int axon_hip_matmul_q8_0_q8(const void* w, const void* xq, float* y, size_t n_out, size_t n_in);
int axon_hip_matmul_q4_0_q8(const void* w, const void* xq, float* y, size_t n_out, size_t n_in);
/* kernels.h:102-110 */
int axon_hip_matmul_q8_0_rows(const void* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
                              size_t y_stride);
int axon_hip_matmul_q4_0_rows(const void* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
                              size_t y_stride);
int axon_hip_matmul_q8_0_q8_rows(const void* w, const void* xq, float* y, size_t n_rows, size_t n_out,
                                 size_t n_in, size_t y_stride);
int axon_hip_matmul_q4_0_q8_rows(const void* w, const void* xq, float* y, size_t n_rows, size_t n_out,
                                 size_t n_in, size_t y_stride);
/* kernels.h:111-112 */
int axon_hip_quantize_row_q8_0(const float* x, void* out, size_t n);
/* kernels.h:114-124 */
int axon_hip_matmul_q4_1(const void* w, const float* x, float* y, size_t n_out, size_t n_in);
int axon_hip_matmul_q4_1_q8(const void* w, const void* xq, float* y, size_t n_out, size_t n_in);
int axon_hip_matmul_q4_1_rows(const void* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
                              size_t y_stride);
int axon_hip_matmul_q4_1_q8_rows(const void* w, const void* xq, float* y, size_t n_rows, size_t n_out,
                                 size_t n_in, size_t y_stride);
/* kernels.h:125-128 */
int axon_hip_matmul_q6_k(const void* w, const float* x, float* y, size_t n_out, size_t n_in);
int axon_hip_matmul_q6_k_rows(const void* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
                              size_t y_stride);

/* ---- Coarse entries of the device-resident forward pass --------------------------------- */

/* The one-time repack of a Q6_K matrix at upload (the GGUF block layout, src/core/dtype.h
 * BlockQ6_K, turned into 16-byte-aligned planes; no counterpart in the reference, which reads
 * the blocks in place). Super-block column c of the [n_out][n_in/256] matrix becomes 13 slices
 * [n_out][16 bytes] (slice s: bytes 16s..16s+15 of each row's block: ql, qh, scales), then the
 * d plane [n_out] of halves padded to 16 bytes. planar_bytes: the copy's size (0 for an n_in
 * that is not a multiple of 256). repack: w (2-byte aligned) into planar (16-byte aligned). */
size_t axon_hip_q6k_planar_bytes(size_t n_out, size_t n_in);
int axon_hip_q6k_repack(const void* w, size_t n_out, size_t n_in, void* planar);
/* matmul_q6_k_rows (kernels.h:125-128) over the planar copy: the same outputs, bit for bit.
 * x 16-byte aligned. */
int axon_hip_matmul_q6_k_planar(const void* planar, const float* x, float* y, size_t n_rows, size_t n_out,
                                size_t n_in, size_t y_stride);
/* One greedy decode step's tail in two launches instead of four (the output matmul of
 * llama.cpp:628, sampler.cpp:100-102's argmax and the next step's embedding_row,
 * llama.cpp:482-485). matmul_q6_k_planar_argmax: axon_hip_matmul_q6_k_planar of one row (the
 * same y, bit for bit) whose workgroups also leave the greedy keys of their outputs in keys
 * (axon_hip_q6k_argmax_parts(n_out) words; key_words must hold them). argmax_embed: the id
 * axon_hip_argmax_rows would choose for the logits row x from those n_keys keys, into *out, and
 * that token's row of the [table_rows][n] embedding table (embedding_rows) into emb. */
size_t axon_hip_q6k_argmax_parts(size_t n_out);
int axon_hip_matmul_q6_k_planar_argmax(const void* planar, const float* x, float* y, size_t n_out, size_t n_in,
                                       uint64_t* keys, size_t key_words);
int axon_hip_argmax_embed(const float* x, const uint64_t* keys, size_t n_keys, int32_t* out, int type,
                          const void* table, size_t table_rows, size_t n, float* emb);
/* Test hook, no counterpart in the reference: which kernel axon_hip_matmul_q6_k_planar runs for
 * one activation row. 0 (the default) chooses by shape; 1 one lane per output row; 2 the
 * products formed by every thread into LDS, then one in-order chain per row (used only where
 * its LDS fits, else as 1); 3 products streamed to the chains through two LDS slots, 64 rows
 * per workgroup. Every path gives the same bits. */
int axon_hip_q6k_force_path(int path);

/* rmsnorm over rows (src/model/llama.cpp:128-134), writing y, its Q8_0 blocks (the next
 * matmul's input, llama.cpp:399-417), or both (either may be NULL). */
int axon_hip_rmsnorm_rows(const float* x, const float* weight, float* y, void* yq, size_t n, size_t n_rows,
                          float eps);
/* quantize_row_q8_0 over rows of n floats, x rows x_stride floats apart (llama.cpp:407-415). */
int axon_hip_quantize_rows_q8_0(const float* x, void* out, size_t n, size_t n_rows, size_t x_stride);
/* silu_mul over rows, optionally quantizing the product to Q8_0 blocks (llama.cpp:600-620). */
int axon_hip_silu_mul_rows(const float* gate, const float* up, float* out, void* outq, size_t n, size_t n_rows);
/* x += y (add_rows, llama.cpp:122-126). */
int axon_hip_add(float* x, const float* y, size_t n);
/* Greedy selection on the device (src/sampling/sampler.cpp:100-102 with the repetition penalty
 * off): out[r] = std::ranges::max_element over row r of x (rows stride floats apart): the first
 * maximum; NaN is skipped, but a NaN first element selects 0. n >= 1. scratch: device words,
 * axon_hip_argmax_scratch_words(n_rows) of them. */
size_t axon_hip_argmax_scratch_words(size_t n_rows);
/* The repetition penalty in place (src/sampling/sampler.cpp:73-97): for each row r, every distinct
 * id in [0, n) among recent[r * recent_stride + i], i < min(recent_len[r], recent_stride), gets
 * logit > 0 ? logit / penalty : logit * penalty, once. recent and recent_len are device arrays
 * holding each row's window (the last repeat_last_n ids), which the caller cuts. */
int axon_hip_repeat_penalty_rows(float* x, size_t n, size_t n_rows, size_t stride, const int32_t* recent,
                                 const uint32_t* recent_len, size_t recent_stride, float penalty);
int axon_hip_argmax_rows(const float* x, size_t n, size_t n_rows, size_t stride, uint64_t* scratch, int32_t* out);
/* argmax_rows without a workspace and without allocating: no counterpart in the reference. For
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). The partial keys live in a fixed device array of
 * AXON_HIP_ARGMAX_NOALLOC_MAX_ROWS * 64 words (256 KiB) that each GPU holds until the process
 * ends; more rows are refused with AXON_HIP_E_INVALID. Every call on one GPU shares that array,
 * so calls that overlap on one GPU (other streams, concurrent graph replays) race. Same ids as
 * axon_hip_argmax_rows. */
#define AXON_HIP_ARGMAX_NOALLOC_MAX_ROWS 512
int axon_hip_argmax_rows_noalloc(const float* x, size_t n, size_t n_rows, size_t stride, int32_t* out);
/* The top-k candidates of the stochastic sampler stages (src/sampling/sampler.cpp:104-118,
 * std::ranges::partial_sort of the ids by logit, descending): row r's k largest values (rows
 * stride floats apart) into out_logit[r * k + i] with their indices in out_id, descending, equal
 * values by ascending index (the reference leaves their order unspecified). NaN is skipped; a
 * row with fewer than k other values ends in ids -1. 1 <= k <= 256, k <= n. */
#define AXON_HIP_MAX_TOPK 256
int axon_hip_topk_rows(const float* x, size_t n, size_t n_rows, size_t stride, size_t k, float* out_logit,
                       int32_t* out_id);
/* Every candidate in order, for top_k 0 or a top_k above 256 (src/sampling/sampler.cpp:105-118,
 * std::ranges::sort of all ids by logit, descending, and the partial_sort whose first top_k it
 * also gives): row r's n values (rows stride floats apart) into out_logit[r * n + i] with their
 * indices in out_id, in the order of axon_hip_topk_rows (descending, equal values by ascending
 * index, -0 equal to +0), the NaN values last with ids -1 and logits 0. work: a device buffer of
 * axon_hip_sort_rows_work_bytes(n, n_rows) bytes. The outputs must not alias x or work. */
size_t axon_hip_sort_rows_work_bytes(size_t n, size_t n_rows);
int axon_hip_sort_rows(const float* x, size_t n, size_t n_rows, size_t stride, void* work, float* out_logit,
                       int32_t* out_id);
/* gate|up with the SwiGLU product and its Q8_0 quantization in one launch (llama.cpp:600-620:
 * out = silu(x W_gate^T) * (x W_up^T), then quantize_row_q8_0 of each row for w_down): the same
 * bits as matmul_q8_fused of the two weights, silu_mul_rows and quantize_rows. out: float
 * [n_rows][n_ff] or NULL; outq: [n_rows][n_ff / 32] Q8_0 blocks, which must not alias xq. n_ff a
 * multiple of 32. AXON_HIP_E_UNSUPPORTED (nothing launched) for up to 64 rows with n_ff below
 * 4096 (too few workgroups), or bases the tile kernel cannot load. */
int axon_hip_matmul_q8_swiglu(int type, const void* xq, size_t n_rows, size_t n_in, const void* w_gate,
                              const void* w_up, size_t n_ff, float* out, void* outq);

/* Y_s[n_rows][n_out_s] (+)= X W_s^T for up to three weights of one type sharing one Q8_0
 * input (mm_fused, llama.cpp:425-472). w[s], y[s] device pointers in host arrays. Rows below
 * 16 run the v_dot4 matvec, 16 and more the int8 MFMA tiles. accumulate adds into y (the
 * residual add fused, llama.cpp:594-595, 621-623). */
int axon_hip_matmul_q8_fused(int type, const void* xq, size_t n_rows, size_t n_in, size_t n_seg,
                             const void* const* w, float* const* y, const size_t* n_out, const size_t* y_stride,
                             int accumulate);

/* rope + Qwen2 bias + KV-cache write over rows (llama.cpp:493-537). */
typedef struct {
  float* q;               /* [rows][q_stride]: n_head heads rotated in place, or NULL */
  float* k;               /* [rows][k_stride]: n_kv heads rotated in place, or NULL */
  float* v;               /* [rows][k_stride]: biased, then copied to the cache, or NULL */
  const float* bq;        /* biases [n_head*head_dim], [n_kv*head_dim] x2, all or none */
  const float* bk;
  const float* bv;
  const int32_t* pos;     /* per-row positions (device), or NULL for pos0 + row */
  int32_t pos0;
  uint32_t q_stride, k_stride;
  uint32_t n_head, n_kv, head_dim, rotary_dim;
  int neox;               /* RopeStyle::NeoX */
  float theta;
  const float* freq_factors; /* device, or NULL */
  const float* table;     /* device cos/sin pairs [pos][rotary_dim/2] built on the host, or NULL */
  void* cache;            /* KV pool base (float or fp16 elements), or NULL for no cache write */
  const int64_t* cache_off; /* per-row element offset of the row's sequence (device), or NULL */
  int64_t k_layer_off, v_layer_off;
  int cache_f16;          /* the cache holds fp16 bit patterns: rows rounded in once, round to nearest
                           * even (CacheType::F16, llama.cpp:525-532, 559-563) */
} axon_hip_rope_rows_args;
int axon_hip_rope_rows(const axon_hip_rope_rows_args* args, size_t n_rows);

/* Ragged grouped-query attention: row r attends over positions [0, n_vis[r]) of its own
 * sequence's K/V rows, found at kv + k_off[r] + k_layer_off and kv + v_off[r] + v_layer_off
 * (elements). One launch serves every sequence of a batch (llama.cpp:539-556) or every query
 * row of a prefill chunk (llama.cpp:566-590). Per-row arrays are device pointers; with them
 * NULL, row r sees n_past + r + 1 positions at the constant offsets. */
typedef struct {
  const float* q;
  float* out;
  uint32_t q_stride, out_stride;
  const void* kv;
  const int64_t* k_off;
  const int64_t* v_off;
  const int32_t* n_vis;
  int64_t k_layer_off, v_layer_off;
  int32_t n_past;
  uint32_t n_head, n_kv, head_dim;
  float scale;
  int f16;                /* the cache holds fp16 bit patterns */
  float* scratch;         /* device score scratch for contexts beyond LDS, or NULL */
  uint32_t max_vis;       /* >= every n_vis */
  void* outq;             /* also the Q8_0 blocks of each output row (wo's input), or NULL */
} axon_hip_attention_rows_args;
int axon_hip_attention_rows(const axon_hip_attention_rows_args* args, size_t n_rows);
/* Floats of scratch axon_hip_attention_rows needs for n_rows rows (0: LDS suffices). Launches
 * of few rows use a two-kernel path whose scores always go through the scratch. */
size_t axon_hip_attention_scratch_floats(const axon_hip_attention_rows_args* args, size_t n_rows);

/* The decode matvec with its neighbours fused in, for 1..4 activation rows of quantized
 * weights (one type for every segment). Input: in_mode 0 Q8_0 blocks (xq), 1 float rows (x,
 * quantized in the kernel as quantize_row_q8_0 does), 2 float rows RMSNorm'd with norm_w and eps
 * first (llama.cpp:500, 598). Output: out_mode 0 y = W x, 1 y += W x (residual), 2 segments gate
 * and up -> y[0] = silu(gate) * up (llama.cpp:600-620), 3 segments q, k, v -> bias, Normal-style
 * RoPE from the cos/sin table at pos[row], q into y[0], k and v into the row's cache slot at
 * cache + cache_off[row] + {k,v}_layer_off + pos * n_out[1] (llama.cpp:493-537). */
typedef struct {
  int type;
  size_t n_seg;
  const void* w[3];
  size_t n_out[3];
  size_t n_rows, n_in;
  int in_mode;
  const void* xq;
  const float* x;
  size_t x_stride;
  const float* norm_w;
  float eps;
  int out_mode;
  float* y[3];
  size_t y_stride[3];
  const float* bias[3];
  const float* rope_table;
  uint32_t rot_half, head_dim;
  const int32_t* pos;
  const int64_t* cache_off;
  void* cache;            /* float or fp16 elements (cache_f16) */
  int64_t k_layer_off, v_layer_off;
  /* out_mode 2 only: also the Q8_0 blocks of every output row (down's input, llama.cpp:600-620,
   * [n_rows][n_out[0] / 32] blocks), or NULL. Requires n_out[0] % 32 == 0. */
  void* outq;
  int cache_f16;          /* out_mode 3: k and v rounded into an fp16 cache (llama.cpp:525-532) */
} axon_hip_matvec_fused_args;
int axon_hip_matvec_fused(const axon_hip_matvec_fused_args* args);
/* 1 when axon_hip_matvec_fused takes this shape (rows, row length, input mode, SiLU pairing). */
int axon_hip_matvec_fused_supported(int type, int in_mode, size_t n_rows, size_t n_in, int silu);
/* q|k|v of 1..64 rows of Q8_0 blocks with the bias, Normal-style RoPE and KV write folded into
 * the int8 MFMA matmul's epilogue (llama.cpp:493-537; replaces matmul_q8_fused followed by
 * rope_rows, kernels/ref/rope.cpp:13-37, with the same bits). The fields of
 * axon_hip_matvec_fused_args with n_seg 3, in_mode 0 (xq) and out_mode 3: q into y[0] (row
 * stride y_stride[0]), k and v into the cache as axon_hip_matvec_fused writes them; norm_w, x
 * and outq are not read. AXON_HIP_E_UNSUPPORTED (nothing launched) above 64 rows or for bases
 * the kernel's dword loads cannot take. */
int axon_hip_matmul_q8_qkv_rope(const axon_hip_matvec_fused_args* args);

/* Every layer of one decode row as a single persistent kernel (llama.cpp:487-623 for a batch of
 * one): per layer, attn_norm, q|k|v, bias, RoPE (Normal style) and the KV write at pos, the
 * attention of every head over positions [0, pos], wo with the residual add, ffn_norm, gate|up,
 * SiLU * up, down with the residual add. The same bits as those steps launched one by one
 * (matvec_fused and attention_rows). One workgroup per CU; a phase's outputs carry the phase's
 * number and their readers poll for it; the caller's stream then continues with the output
 * norm and matrix. F32 or fp16 cache, head
 * size 64, n_embd a multiple of 32 up to 2048, Q8_0 / Q4_0 / Q4_1 layer matrices (one type per
 * matrix role); axon_hip_decode_layers_unsupported names what else it needs. */
typedef struct {
  const void* wq;
  const void* wk;
  const void* wv;
  const void* wo;
  const void* w_gate;
  const void* w_up;
  const void* w_down;
  const float* attn_norm;
  const float* ffn_norm;
  const float* bq; /* Q/K/V biases, all or none */
  const float* bk;
  const float* bv;
  int64_t k_layer_off, v_layer_off; /* cache elements from a sequence's slot to this layer's K / V rows */
} axon_hip_decode_layer;

typedef struct {
  uint32_t n_layer, n_embd, n_head, n_head_kv, n_ff, rotary_dim;
  int type_qkv, type_o, type_gate_up, type_down;
  uint32_t max_ctx; /* positions of a cache slot: calls take pos < max_ctx */
  int cache_f16;    /* 1: the KV pool holds fp16 bit patterns (llama.cpp:525-532), else floats */
} axon_hip_decode_shape;

typedef struct {
  const axon_hip_decode_layer* layers; /* device array of n_layer records */
  float eps, scale;                    /* RMSNorm epsilon; 1 / sqrt(head size) */
  const float* rope_table;             /* device (cos, sin) [pos][rotary_dim / 2], built on the host */
  float* x;                            /* device [n_embd]: the row's residual stream, in and out */
  float* cache;                        /* device KV pool (float elements, or fp16 with shape->cache_f16) */
  int64_t cache_off;                   /* the row's slot, in elements */
  int32_t pos;                         /* the row's position */
  void* work;                          /* device workspace, zeroed once before its first call */
  uint64_t* epoch;                     /* host: phases run on this workspace, updated by the call */
  uint32_t* status;                    /* pinned host word, 0 at the start: nonzero once a call gave up */
} axon_hip_decode_layers_args;

/* Test hook, no counterpart in the reference: the polls of one tagged word after which a
 * workgroup of later axon_hip_decode_layers calls gives up (0 restores the default, about a
 * second). A small limit forces the give-up path from the host: the kernel still drains, the
 * call's status word is set, and the caller's recovery runs. */
int axon_hip_decode_layers_set_spin_limit(uint32_t polls);
/* Test hook, no counterpart in the reference: with on nonzero, no wait of later
 * axon_hip_decode_layers calls sees its word as written, so every workgroup gives up after the
 * spin limit's polls whatever the timing (with a small limit, at once): the give-up path runs
 * deterministically. 0 restores normal waits. */
int axon_hip_decode_layers_set_fail_waits(int on);
/* Measurement hook, no counterpart in the reference: with a device buffer of
 * axon_hip_decode_layers_stamp_count(shape, &ticks_per_second) uint64 words, every later
 * axon_hip_decode_layers call records the device's constant-rate clock (s_memrealtime) at four points of every phase of every layer in every
 * workgroup, each call overwriting the last: word ((layer * 5 + phase) * 4 + point) * CUs +
 * workgroup, phases A (norm, q|k|v, RoPE, cache row), B (attention), C (wo), D (norm, gate|up,
 * SiLU), E (down); points: the phase's start, its first inputs in (every thread's polls done),
 * its second inputs in (B: the scores; else the same as the first), its end. A shape small
 * enough to run on 128 workgroups runs on 128 (then the words of workgroups 128 and up keep
 * what they held). NULL turns it off. The instrumented launch adds one workgroup barrier per
 * poll. */
int axon_hip_decode_layers_set_stamps(uint64_t* stamps);
size_t axon_hip_decode_layers_stamp_count(const axon_hip_decode_shape* shape, double* ticks_per_second);
size_t axon_hip_decode_layers_workspace_bytes(const axon_hip_decode_shape* shape);
/* NULL when this device runs the shape, else the reason. */
const char* axon_hip_decode_layers_unsupported(const axon_hip_decode_shape* shape);
/* Refuses (AXON_HIP_E_HIP) while *status is nonzero: a previous call gave up waiting for
 * another workgroup's output after about a second of polling, its results are void, and the
 * workspace must be zeroed again and *epoch, *status reset before the next call. */
int axon_hip_decode_layers(const axon_hip_decode_shape* shape, const axon_hip_decode_layers_args* args);

/* embedding_row for a device array of token ids (llama.cpp:482-485). */
int axon_hip_embedding_rows(int type, const void* table, size_t n, const int32_t* ids, size_t n_rows, float* out);

/* Test hook: per-block int32 sums of one weight row against one Q8_0 activation row, the
 * integer phase of matmul_*_q8 (src/kernels/ref/quant.cpp:47-50, 59-65, 166-175); sumx (Q4_1
 * only, else may be NULL) receives the activation's quant sum per block. */
int axon_hip_block_sums(int type, const void* w_row, const void* xq, size_t n_blocks, int32_t* sumi,
                        int32_t* sumx);

#ifdef __cplusplus
}
#endif
#endif
