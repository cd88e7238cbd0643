/*
 * TEST INFRASTRUCTURE ONLY (the CPU oracle; see oracle.h). A plain-C restatement of the
 * reference scalar kernel table. Each function names the reference lines it follows.
 * Build with -ffp-contract=off: the x86 scalar table multiplies and adds separately.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

/* ---- conversions: src/core/dtype.cpp:198-286 ------------------------------------------- */

static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* dtype.cpp:198-223: exact widening, subnormals renormalised, inf/nan payload kept. */
float ora_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exponent = (h >> 10) & 0x1Fu;
  const uint32_t mantissa = h & 0x3FFu;
  uint32_t out;
  if (exponent == 0) {
    if (mantissa == 0) {
      out = sign;
    } else {
      uint32_t m = mantissa, e = 127 - 15 + 1;
      while ((m & 0x400u) == 0) { m <<= 1; --e; }
      m &= 0x3FFu;
      out = sign | (e << 23) | (m << 13);
    }
  } else if (exponent == 0x1F) {
    out = sign | 0x7F800000u | (mantissa << 13);
  } else {
    out = sign | ((exponent + (127 - 15)) << 23) | (mantissa << 13);
  }
  return f32_from_bits(out);
}

/* dtype.cpp:225-272: round to nearest even, subnormal halves, overflow to inf. */
uint16_t ora_fp32_to_fp16(float value) {
  const uint32_t bits = bits_from_f32(value);
  const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  const uint32_t exponent = (bits >> 23) & 0xFFu;
  const uint32_t mantissa = bits & 0x7FFFFFu;
  if (exponent == 0xFF) {
    const uint16_t payload = (uint16_t)(mantissa >> 13);
    return (uint16_t)(sign | 0x7C00u | (mantissa != 0 && payload == 0 ? 1u : payload));
  }
  const int unbiased = (int)exponent - 127;
  if (unbiased > 15) return (uint16_t)(sign | 0x7C00u);
  if (unbiased >= -14) {
    uint32_t half_exp = (uint32_t)(unbiased + 15);
    uint32_t half_man = mantissa >> 13;
    const uint32_t rest = mantissa & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (half_man & 1u) != 0)) {
      ++half_man;
      if (half_man == 0x400u) {
        half_man = 0;
        ++half_exp;
        if (half_exp == 0x1F) return (uint16_t)(sign | 0x7C00u);
      }
    }
    return (uint16_t)(sign | (half_exp << 10) | half_man);
  }
  if (unbiased >= -25) {
    const uint32_t full = mantissa | 0x800000u;
    const int shift = -14 - unbiased + 13;
    uint32_t half_man = full >> shift;
    const uint32_t rest = full & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rest > halfway || (rest == halfway && (half_man & 1u) != 0)) ++half_man;
    return (uint16_t)(sign | half_man);
  }
  return sign;
}

/* dtype.cpp:274-286 */
float ora_bf16_to_fp32(uint16_t bits) { return f32_from_bits((uint32_t)bits << 16); }

uint16_t ora_fp32_to_bf16(float value) {
  const uint32_t bits = bits_from_f32(value);
  if (((bits >> 23) & 0xFFu) == 0xFFu && (bits & 0x7FFFFFu) != 0) {
    return (uint16_t)((bits >> 16) | 0x40u);
  }
  const uint32_t lsb = (bits >> 16) & 1u;
  return (uint16_t)((bits + 0x7FFFu + lsb) >> 16);
}

/* ---- block conversions: dtype.cpp:288-354 ----------------------------------------------- */

void ora_dequantize_block_q8_0(const ora_block_q8_0* b, float* out) {
  const float d = ora_fp16_to_fp32(b->d);
  for (int i = 0; i < 32; ++i) out[i] = (float)b->qs[i] * d;
}

void ora_dequantize_block_q4_0(const ora_block_q4_0* b, float* out) {
  const float d = ora_fp16_to_fp32(b->d);
  for (int i = 0; i < 16; ++i) {
    out[i] = (float)((int)(b->qs[i] & 0x0F) - 8) * d;
    out[i + 16] = (float)((int)(b->qs[i] >> 4) - 8) * d;
  }
}

void ora_dequantize_block_q4_1(const ora_block_q4_1* b, float* out) {
  const float d = ora_fp16_to_fp32(b->d);
  const float m = ora_fp16_to_fp32(b->m);
  for (int i = 0; i < 16; ++i) {
    out[i] = (float)(b->qs[i] & 0x0F) * d + m;
    out[i + 16] = (float)(b->qs[i] >> 4) * d + m;
  }
}

/* dtype.cpp:312-336: ggml's order (d * scale) * q, four 32-element strips per 128. */
void ora_dequantize_block_q6_k(const ora_block_q6_k* b, float* out) {
  const float d = ora_fp16_to_fp32(b->d);
  const uint8_t* ql = b->ql;
  const uint8_t* qh = b->qh;
  const int8_t* sc = b->scales;
  float* y = out;
  for (int n = 0; n < 256; n += 128) {
    for (int l = 0; l < 32; ++l) {
      const int is = l / 16;
      const int q1 = (int)((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32;
      const int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
      const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
      const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
      y[l] = d * (float)sc[is] * (float)q1;
      y[l + 32] = d * (float)sc[is + 2] * (float)q2;
      y[l + 64] = d * (float)sc[is + 4] * (float)q3;
      y[l + 96] = d * (float)sc[is + 6] * (float)q4;
    }
    y += 128;
    ql += 64;
    qh += 32;
    sc += 8;
  }
}

/* dtype.cpp:338-354: amax, d = amax / 127, id = 1/d (0 for an all-zero block), q = roundf. */
void ora_quantize_row_q8_0(const float* x, ora_block_q8_0* out, size_t n) {
  for (size_t b = 0; b < n / 32; ++b) {
    const float* block = x + b * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
      const float a = fabsf(block[i]);
      amax = a > amax ? a : amax;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    out[b].d = ora_fp32_to_fp16(d);
    for (int i = 0; i < 32; ++i) out[b].qs[i] = (int8_t)roundf(block[i] * id);
  }
}

/* ---- float matmuls: src/kernels/ref/matmul.cpp:12-68 ------------------------------------ */

void ora_matmul_f32(const float* w, const float* x, float* y, size_t n_out, size_t n_in) {
  for (size_t o = 0; o < n_out; ++o) {
    const float* row = w + o * n_in;
    float acc = 0.0f;
    for (size_t i = 0; i < n_in; ++i) acc += row[i] * x[i];
    y[o] = acc;
  }
}

void ora_matmul_f16(const uint16_t* w, const float* x, float* y, size_t n_out, size_t n_in) {
  for (size_t o = 0; o < n_out; ++o) {
    const uint16_t* row = w + o * n_in;
    float acc = 0.0f;
    for (size_t i = 0; i < n_in; ++i) acc += ora_fp16_to_fp32(row[i]) * x[i];
    y[o] = acc;
  }
}

void ora_matmul_bf16(const uint16_t* w, const float* x, float* y, size_t n_out, size_t n_in) {
  for (size_t o = 0; o < n_out; ++o) {
    const uint16_t* row = w + o * n_in;
    float acc = 0.0f;
    for (size_t i = 0; i < n_in; ++i) acc += ora_bf16_to_fp32(row[i]) * x[i];
    y[o] = acc;
  }
}

void ora_matmul_f32_rows(const float* w, const float* x, float* y, size_t n_rows, size_t n_out,
                         size_t n_in, size_t y_stride) {
  for (size_t r = 0; r < n_rows; ++r) ora_matmul_f32(w, x + r * n_in, y + r * y_stride, n_out, n_in);
}

void ora_matmul_f16_rows(const uint16_t* w, const float* x, float* y, size_t n_rows, size_t n_out,
                         size_t n_in, size_t y_stride) {
  for (size_t r = 0; r < n_rows; ++r) ora_matmul_f16(w, x + r * n_in, y + r * y_stride, n_out, n_in);
}

void ora_matmul_bf16_rows(const uint16_t* w, const float* x, float* y, size_t n_rows, size_t n_out,
                          size_t n_in, size_t y_stride) {
  for (size_t r = 0; r < n_rows; ++r) ora_matmul_bf16(w, x + r * n_in, y + r * y_stride, n_out, n_in);
}

/* ---- elementwise: ref/rmsnorm.cpp:10-21, ref/rope.cpp:13-37, ref/softmax.cpp:10-25,
 *      ref/silu.cpp:8-13 -------------------------------------------------------------------- */

void ora_rmsnorm(const float* x, const float* weight, float* y, size_t n, float eps) {
  double sum_squares = 0.0;
  for (size_t i = 0; i < n; ++i) sum_squares += (double)x[i] * (double)x[i];
  const float inv_rms = (float)(1.0 / sqrt(sum_squares / (double)n + (double)eps));
  for (size_t i = 0; i < n; ++i) y[i] = x[i] * inv_rms * weight[i];
}

void ora_rope(float* x, size_t n_heads, size_t pos, size_t head_dim, size_t rotary_dim, float theta,
              int style, const float* freq_factors) {
  const size_t half = rotary_dim / 2;
  const double th = (double)theta;
  const double rd = (double)rotary_dim;
  for (size_t i = 0; i < half; ++i) {
    double inv_freq = pow(th, -(double)(2 * i) / rd);
    if (freq_factors != NULL) inv_freq /= (double)freq_factors[i];
    const double angle = (double)pos * inv_freq;
    const float c = (float)cos(angle);
    const float s = (float)sin(angle);
    const size_t a = style == 0 ? 2 * i : i;
    const size_t b = style == 0 ? 2 * i + 1 : i + half;
    for (size_t h = 0; h < n_heads; ++h) {
      float* head = x + h * head_dim;
      const float x0 = head[a];
      const float x1 = head[b];
      head[a] = x0 * c - x1 * s;
      head[b] = x0 * s + x1 * c;
    }
  }
}

void ora_softmax(float* x, size_t n) {
  float max = x[0];
  for (size_t i = 1; i < n; ++i) max = x[i] > max ? x[i] : max;
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) {
    x[i] = expf(x[i] - max);
    sum += (double)x[i];
  }
  const float inv_sum = (float)(1.0 / sum);
  for (size_t i = 0; i < n; ++i) x[i] *= inv_sum;
}

void ora_silu_mul(const float* gate, const float* up, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float g = gate[i];
    out[i] = g / (1.0f + expf(-g)) * up[i];
  }
}

/* ref/embedding.cpp:12-64 */
void ora_embedding_row(int type, const void* table, size_t n, int64_t index, float* out) {
  const size_t row = (size_t)index;
  switch (type) {
  case ORA_F32:
    memcpy(out, (const float*)table + row * n, n * sizeof(float));
    return;
  case ORA_F16: {
    const uint16_t* src = (const uint16_t*)table + row * n;
    for (size_t i = 0; i < n; ++i) out[i] = ora_fp16_to_fp32(src[i]);
    return;
  }
  case ORA_BF16: {
    const uint16_t* src = (const uint16_t*)table + row * n;
    for (size_t i = 0; i < n; ++i) out[i] = ora_bf16_to_fp32(src[i]);
    return;
  }
  case ORA_Q8_0: {
    const ora_block_q8_0* src = (const ora_block_q8_0*)table + row * (n / 32);
    for (size_t b = 0; b < n / 32; ++b) ora_dequantize_block_q8_0(src + b, out + b * 32);
    return;
  }
  case ORA_Q4_0: {
    const ora_block_q4_0* src = (const ora_block_q4_0*)table + row * (n / 32);
    for (size_t b = 0; b < n / 32; ++b) ora_dequantize_block_q4_0(src + b, out + b * 32);
    return;
  }
  case ORA_Q4_1: {
    const ora_block_q4_1* src = (const ora_block_q4_1*)table + row * (n / 32);
    for (size_t b = 0; b < n / 32; ++b) ora_dequantize_block_q4_1(src + b, out + b * 32);
    return;
  }
  case ORA_Q6_K: {
    const ora_block_q6_k* src = (const ora_block_q6_k*)table + row * (n / 256);
    for (size_t b = 0; b < n / 256; ++b) ora_dequantize_block_q6_k(src + b, out + b * 256);
    return;
  }
  default:
    return;
  }
}

/* ---- attention: ref/attention.cpp:12-113 ------------------------------------------------ */

static float dot_f32(const float* a, const float* b, size_t n) {
  float acc = 0.0f;
  for (size_t i = 0; i < n; ++i) acc += a[i] * b[i];
  return acc;
}

void ora_attention_kv_heads(const float* q, const float* k_cache, const float* v_cache, float* out,
                            float* scores, size_t n_q, size_t n_past, size_t n_head,
                            size_t n_head_kv, size_t head_dim, float scale, size_t head_begin,
                            size_t head_end) {
  const size_t group = n_head / n_head_kv;
  const size_t total = n_past + n_q;
  for (size_t h = head_begin; h < head_end; ++h) {
    const size_t kv_head = h / group;
    for (size_t i = 0; i < n_q; ++i) {
      const size_t pos = n_past + i;
      float* row = scores + i * total;
      const float* q_i = q + (i * n_head + h) * head_dim;
      for (size_t j = 0; j <= pos; ++j) {
        row[j] = scale * dot_f32(q_i, k_cache + (j * n_head_kv + kv_head) * head_dim, head_dim);
      }
      ora_softmax(row, pos + 1);
      float* o = out + (i * n_head + h) * head_dim;
      for (size_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
      for (size_t j = 0; j <= pos; ++j) {
        const float* v_j = v_cache + (j * n_head_kv + kv_head) * head_dim;
        for (size_t d = 0; d < head_dim; ++d) o[d] += row[j] * v_j[d];
      }
    }
  }
}

void ora_attention_kv(const float* q, const float* k_cache, const float* v_cache, float* out,
                      float* scores, size_t n_q, size_t n_past, size_t n_head, size_t n_head_kv,
                      size_t head_dim, float scale) {
  ora_attention_kv_heads(q, k_cache, v_cache, out, scores, n_q, n_past, n_head, n_head_kv, head_dim,
                         scale, 0, n_head);
}

void ora_attention(const float* q, const float* k, const float* v, float* out, float* scores,
                   size_t seq, size_t n_head, size_t n_head_kv, size_t head_dim, float scale) {
  ora_attention_kv(q, k, v, out, scores, seq, 0, n_head, n_head_kv, head_dim, scale);
}

void ora_attention_kv_heads_f16(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                float* out, float* scores, size_t n_q, size_t n_past, size_t n_head,
                                size_t n_head_kv, size_t head_dim, float scale, size_t head_begin,
                                size_t head_end) {
  const size_t group = n_head / n_head_kv;
  const size_t total = n_past + n_q;
  for (size_t h = head_begin; h < head_end; ++h) {
    const size_t kv_head = h / group;
    for (size_t i = 0; i < n_q; ++i) {
      const size_t pos = n_past + i;
      float* row = scores + i * total;
      const float* q_i = q + (i * n_head + h) * head_dim;
      for (size_t j = 0; j <= pos; ++j) {
        const uint16_t* k_j = k_cache + (j * n_head_kv + kv_head) * head_dim;
        float acc = 0.0f;
        for (size_t d = 0; d < head_dim; ++d) acc += q_i[d] * ora_fp16_to_fp32(k_j[d]);
        row[j] = scale * acc;
      }
      ora_softmax(row, pos + 1);
      float* o = out + (i * n_head + h) * head_dim;
      for (size_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
      for (size_t j = 0; j <= pos; ++j) {
        const uint16_t* v_j = v_cache + (j * n_head_kv + kv_head) * head_dim;
        for (size_t d = 0; d < head_dim; ++d) o[d] += row[j] * ora_fp16_to_fp32(v_j[d]);
      }
    }
  }
}

/* ---- quantized matmuls: src/kernels/ref/quant.cpp:13-247 -------------------------------- */

static float dot_q8_0_f32(const ora_block_q8_0* row, const float* x, size_t nb) {
  float acc = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const float d = ora_fp16_to_fp32(row[b].d);
    const float* xb = x + b * 32;
    for (int i = 0; i < 32; ++i) acc += (float)row[b].qs[i] * d * xb[i];
  }
  return acc;
}

static float dot_q4_0_f32(const ora_block_q4_0* row, const float* x, size_t nb) {
  float acc = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const float d = ora_fp16_to_fp32(row[b].d);
    const float* xb = x + b * 32;
    for (int i = 0; i < 16; ++i) {
      const float low = (float)((int)(row[b].qs[i] & 0x0F) - 8);
      const float high = (float)((int)(row[b].qs[i] >> 4) - 8);
      acc += low * d * xb[i];
      acc += high * d * xb[i + 16];
    }
  }
  return acc;
}

static float dot_q4_1_f32(const ora_block_q4_1* row, const float* x, size_t nb) {
  float acc = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const float d = ora_fp16_to_fp32(row[b].d);
    const float m = ora_fp16_to_fp32(row[b].m);
    const float* xb = x + b * 32;
    for (int i = 0; i < 16; ++i) {
      acc += ((float)(row[b].qs[i] & 0x0F) * d + m) * xb[i];
      acc += ((float)(row[b].qs[i] >> 4) * d + m) * xb[i + 16];
    }
  }
  return acc;
}

static int32_t sumi_q8_0(const ora_block_q8_0* w, const ora_block_q8_0* x) {
  int32_t sumi = 0;
  for (int i = 0; i < 32; ++i) sumi += (int32_t)w->qs[i] * (int32_t)x->qs[i];
  return sumi;
}

static int32_t sumi_q4_0(const ora_block_q4_0* w, const ora_block_q8_0* x) {
  int32_t sumi = 0;
  for (int i = 0; i < 16; ++i) {
    const int low = (int)(w->qs[i] & 0x0F) - 8;
    const int high = (int)(w->qs[i] >> 4) - 8;
    sumi += low * (int32_t)x->qs[i];
    sumi += high * (int32_t)x->qs[i + 16];
  }
  return sumi;
}

static void sumi_q4_1(const ora_block_q4_1* w, const ora_block_q8_0* x, int32_t* si, int32_t* sx) {
  int32_t sumi = 0, sumx = 0;
  for (int i = 0; i < 16; ++i) {
    const int low = (int)(w->qs[i] & 0x0F);
    const int high = (int)(w->qs[i] >> 4);
    sumi += low * (int32_t)x->qs[i] + high * (int32_t)x->qs[i + 16];
    sumx += (int32_t)x->qs[i] + (int32_t)x->qs[i + 16];
  }
  *si = sumi;
  *sx = sumx;
}

static float dot_q8_0_q8(const ora_block_q8_0* row, const ora_block_q8_0* xq, size_t nb) {
  float acc = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const int32_t sumi = sumi_q8_0(row + b, xq + b);
    acc += (float)sumi * ora_fp16_to_fp32(row[b].d) * ora_fp16_to_fp32(xq[b].d);
  }
  return acc;
}

static float dot_q4_0_q8(const ora_block_q4_0* row, const ora_block_q8_0* xq, size_t nb) {
  float acc = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const int32_t sumi = sumi_q4_0(row + b, xq + b);
    acc += (float)sumi * ora_fp16_to_fp32(row[b].d) * ora_fp16_to_fp32(xq[b].d);
  }
  return acc;
}

/* quant.cpp:163-181: acc += sumi*d*dx + m*dx*sumx, the right side summed before the add. */
static float dot_q4_1_q8(const ora_block_q4_1* row, const ora_block_q8_0* xq, size_t nb) {
  float acc = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    int32_t sumi, sumx;
    sumi_q4_1(row + b, xq + b, &sumi, &sumx);
    const float dx = ora_fp16_to_fp32(xq[b].d);
    acc += (float)sumi * ora_fp16_to_fp32(row[b].d) * dx +
           ora_fp16_to_fp32(row[b].m) * dx * (float)sumx;
  }
  return acc;
}

static float dot_q6_k_f32(const ora_block_q6_k* row, const float* x, size_t nb) {
  float acc = 0.0f;
  float values[256];
  for (size_t b = 0; b < nb; ++b) {
    ora_dequantize_block_q6_k(row + b, values);
    const float* xb = x + b * 256;
    for (int i = 0; i < 256; ++i) acc += values[i] * xb[i];
  }
  return acc;
}

void ora_block_sums(int type, const void* w_row, const ora_block_q8_0* xq, size_t n_blocks,
                    int32_t* sumi, int32_t* sumx) {
  for (size_t b = 0; b < n_blocks; ++b) {
    if (type == ORA_Q8_0) {
      sumi[b] = sumi_q8_0((const ora_block_q8_0*)w_row + b, xq + b);
    } else if (type == ORA_Q4_0) {
      sumi[b] = sumi_q4_0((const ora_block_q4_0*)w_row + b, xq + b);
    } else {
      int32_t sx;
      sumi_q4_1((const ora_block_q4_1*)w_row + b, xq + b, &sumi[b], &sx);
      if (sumx != NULL) sumx[b] = sx;
    }
  }
}

#define ORA_MATMUL(name, wtype, xtype, dotfn)                                                    \
  void ora_##name(const wtype* w, const xtype* x, float* y, size_t n_out, size_t n_in) {          \
    const size_t nb = n_in / 32;                                                                  \
    for (size_t o = 0; o < n_out; ++o) y[o] = dotfn(w + o * nb, x, nb);                           \
  }

ORA_MATMUL(matmul_q8_0, ora_block_q8_0, float, dot_q8_0_f32)
ORA_MATMUL(matmul_q4_0, ora_block_q4_0, float, dot_q4_0_f32)
ORA_MATMUL(matmul_q4_1, ora_block_q4_1, float, dot_q4_1_f32)
ORA_MATMUL(matmul_q8_0_q8, ora_block_q8_0, ora_block_q8_0, dot_q8_0_q8)
ORA_MATMUL(matmul_q4_0_q8, ora_block_q4_0, ora_block_q8_0, dot_q4_0_q8)
ORA_MATMUL(matmul_q4_1_q8, ora_block_q4_1, ora_block_q8_0, dot_q4_1_q8)

void ora_matmul_q6_k(const ora_block_q6_k* w, const float* x, float* y, size_t n_out, size_t n_in) {
  const size_t nb = n_in / 256;
  for (size_t o = 0; o < n_out; ++o) y[o] = dot_q6_k_f32(w + o * nb, x, nb);
}

/* The float-activation rows entries step n_in floats per row (quant.cpp:111-123, 219-224,
 * 242-247); the Q8_0-activation ones step n_in / 32 blocks (quant.cpp:125-139, 226-232). */
#define ORA_ROWS_F(name, single, wtype)                                                            \
  void ora_##name(const wtype* w, const float* x, float* y, size_t n_rows, size_t n_out,            \
                  size_t n_in, size_t y_stride) {                                                 \
    for (size_t r = 0; r < n_rows; ++r) ora_##single(w, x + r * n_in, y + r * y_stride, n_out, n_in); \
  }
#define ORA_ROWS_Q(name, single, wtype)                                                            \
  void ora_##name(const wtype* w, const ora_block_q8_0* xq, float* y, size_t n_rows, size_t n_out,  \
                  size_t n_in, size_t y_stride) {                                                 \
    const size_t nb = n_in / 32;                                                                  \
    for (size_t r = 0; r < n_rows; ++r) ora_##single(w, xq + r * nb, y + r * y_stride, n_out, n_in); \
  }

ORA_ROWS_F(matmul_q8_0_rows, matmul_q8_0, ora_block_q8_0)
ORA_ROWS_F(matmul_q4_0_rows, matmul_q4_0, ora_block_q4_0)
ORA_ROWS_F(matmul_q4_1_rows, matmul_q4_1, ora_block_q4_1)
ORA_ROWS_F(matmul_q6_k_rows, matmul_q6_k, ora_block_q6_k)
ORA_ROWS_Q(matmul_q8_0_q8_rows, matmul_q8_0_q8, ora_block_q8_0)
ORA_ROWS_Q(matmul_q4_0_q8_rows, matmul_q4_0_q8, ora_block_q4_0)
ORA_ROWS_Q(matmul_q4_1_q8_rows, matmul_q4_1_q8, ora_block_q4_1)
