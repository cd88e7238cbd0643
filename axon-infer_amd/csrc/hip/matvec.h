// Launch descriptors shared between the kernel translation units and the C ABI layer.
#pragma once

#include <cstdint>

namespace axon_hip {

// One weight of a fused matvec launch: rows [0, n_out) of w, written to y[m * y_stride + o].
struct MatvecSeg {
  const uint8_t* w;
  float* y;
  uint32_t n_out;
  uint32_t y_stride;
  uint32_t wg_begin;  // first workgroup of this segment (filled by the launcher)
};

struct MatvecArgs {
  MatvecSeg seg[3];
  const uint8_t* xq;  // [m][nb] Q8_0 blocks (Q8_0-activation paths) or [m][n_in] floats
  uint32_t nb;        // blocks (or super-blocks) per weight row
  uint32_t m;         // activation rows in this launch
  uint32_t rows;      // weight rows per workgroup (filled by the launcher)
  uint32_t lds_tile;  // LDS byte offsets (filled by the launcher)
  uint32_t lds_scratch;
  int n_seg;
  int accumulate;     // y += W x instead of y = W x
  uint8_t* outq;      // the SwiGLU tile path: Q8_0 blocks of each output row
  uint64_t* argmax_part;  // one-row planar Q6_K: each workgroup's greedy key of its outputs, or null
};

// The fused decode matvec (matvec_fused.hip): input prologue and output epilogue modes.
enum FusedIn : int { kInQ8 = 0, kInF32 = 1, kInNorm = 2 };
enum FusedOut : int { kOutStore = 0, kOutAdd = 1, kOutSilu = 2, kOutRope = 3 };

struct FusedArgs {
  const uint8_t* w[3];
  uint32_t n_out[3];
  uint32_t wg_begin[3];  // filled by the launcher
  int n_seg;
  uint32_t nb, m;
  uint32_t rows, lds_tile, lds_scratch;  // filled by the launcher
  uint32_t lds_stage;                    // filled by the launcher (staged-prologue kernel)
  int in_mode;
  const uint8_t* xq;      // kInQ8: [m][nb] blocks
  const float* x;         // kInF32 / kInNorm: [m][x_stride] floats
  uint32_t x_stride;
  const float* norm_w;    // kInNorm
  float eps;
  int out_mode;
  float* y[3];
  uint32_t y_stride[3];
  const float* bias[3];   // kOutRope: per segment, or null
  const float* rope_table;
  uint32_t rot_half, head_dim;
  const int32_t* pos;     // per activation row (device)
  const int64_t* cache_off;
  void* cache;            // kOutRope: float or fp16 elements (cache_f16)
  int64_t k_layer_off, v_layer_off;
  uint8_t* outq;          // kOutSilu: also [m][n_out / 32] Q8_0 blocks of the output, or null
  int cache_f16;
};

bool matvec_fused_fits(int type, int in_mode, uint32_t m, uint32_t nb, bool silu);
int matvec_fused_launch(int type, FusedArgs& a);

// The q|k|v epilogue of the few-rows MFMA kernel (rope_rows_kernel's work, for three segments
// q, k, v): per segment bias (or null), Normal-style RoPE over the first rot_half pairs of each
// head at pos[row] from the cos/sin table, q into seg[0].y, k and v into the cache at
// cache_off[row] + {k,v}_layer_off + pos * kv_row (float elements, or fp16 with cache_f16).
struct RowsRope {
  const float* bias[3];
  const float* table;
  const int32_t* pos;
  const int64_t* cache_off;
  void* cache;
  int64_t k_layer_off, v_layer_off;
  uint32_t rot_half, head_dim, kv_row;
  int cache_f16;
};

// Quantized weights (Q8_0 / Q4_0 / Q4_1) against Q8_0 activations, m <= 4 rows.
int matvec_q8_launch(int type, MatvecArgs& a);
// The most activation rows (1..4) one matvec launch takes at nb blocks per row.
uint32_t matvec_q8_max_rows(int type, uint32_t nb);
// Q6_K weights against float activations, any m (launched in groups that fit LDS).
int matvec_q6k_launch(MatvecArgs& a, uint32_t n_in);
// The planar Q6_K layout (matvec_q6k.hip): bytes per super-block column, the one-time repack
// from native blocks, and the matvec over it (seg[0].w the planar copy).
size_t q6k_planar_column_bytes(uint32_t n_out);
int q6k_repack_launch(const uint8_t* src, uint8_t* dst, uint32_t n_out, uint32_t nsb);
int matvec_q6k_planar_launch(MatvecArgs& a, uint32_t n_in);
// With a.argmax_part set (one activation row): the one-lane-per-row kernel, which also leaves
// q6k_planar_argmax_parts(n_out) greedy keys (argmax_key of each workgroup's first maximum).
uint32_t q6k_planar_argmax_parts(uint32_t n_out);
// Test hook: 0 chooses the one-row kernel by shape; 1 the one-lane-per-row kernel, 2 the
// products-then-chains kernel (where its LDS fits), 3 the streamed-ring kernel.
void matvec_q6k_force_path(int path);
// q|k|v of 1..kRowsMaxM rows on the few-rows MFMA kernel with the RowsRope epilogue
// (kUnsupported, nothing launched, where matmul_q8_rows_fits refuses the shape).
int matmul_q8_rows_rope_launch(int type, MatvecArgs& a, const RowsRope& rp);
// int8 MFMA tiles for 16 or more Q8_0 activation rows.
int matmul_q8_mfma_launch(int type, MatvecArgs& a);
// int8 MFMA for 1..kRowsMaxM activation rows (batched decode): every segment in one grid, one
// 16 x 16 tile per wave; the same outputs, bit for bit, as the other Q8_0-activation paths.
constexpr uint32_t kRowsMaxM = 64;
// many_rows: the prefill tile kernel's bounds (any row count) instead of 1..kRowsMaxM.
bool matmul_q8_rows_fits(int type, const MatvecArgs& a, bool many_rows = false);
int matmul_q8_rows_launch(int type, MatvecArgs& a);
// int8 MFMA for 65 and more activation rows (prefill, mixed passes): TN x 64 tiles, every
// segment in one grid, the same per-output order.
int matmul_q8_tile_launch(int type, MatvecArgs& a);
// 33..64 rows on matrices of at least 128 tiles of 64 weight rows: the tile kernel reads the
// weights once where the few-rows kernel's 16-row tiles read them up to four times.
bool matmul_q8_tile_fills(const MatvecArgs& a);
// gate|up with the SwiGLU product and its Q8_0 blocks in the epilogue: seg[0] gate (y: the float
// product, or null), seg[1] up, outq the blocks; n_out a multiple of 32.
int matmul_q8_swiglu_launch(int type, MatvecArgs& a);

}  // namespace axon_hip
