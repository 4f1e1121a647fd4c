/*
 * it_oracle.c -- CPU oracle for the KV-cache hot path (TEST INFRASTRUCTURE).
 *
 * A plain-C restatement of the reference crate's CPU arithmetic, used only
 * as the checker for the HIP library (tests/, smoke()) and as bench.py's CPU
 * baseline.  Never linked into the product library.  Built with
 * -O2 -ffp-contract=off and no fast-math so that every a*b+c rounds twice, as
 * the Rust reference does.  Reference paths are relative to the reference
 * crate root.
 */
#include "it_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Seeded synthetic inputs (test plumbing, no reference counterpart).        */
/* ------------------------------------------------------------------------ */
uint64_t orc_splitmix64(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static double u01_open(uint64_t* st) {
  /* (0, 1]: never 0 so log() is finite. */
  return ((double)(orc_splitmix64(st) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void orc_fill_normal_f32(uint64_t seed, float* out, size_t n) {
  uint64_t st = seed;
  const double two_pi = 6.283185307179586476925286766559;
  size_t i = 0;
  while (i < n) {
    double u1 = u01_open(&st), u2 = u01_open(&st);
    double r = sqrt(-2.0 * log(u1));
    out[i++] = (float)(r * cos(two_pi * u2));
    if (i < n) out[i++] = (float)(r * sin(two_pi * u2));
  }
}

void orc_fill_uniform_i32(uint64_t seed, int32_t lo, int32_t hi, int32_t* out, size_t n) {
  uint64_t st = seed;
  uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
  for (size_t i = 0; i < n; ++i) out[i] = (int32_t)((int64_t)lo + (int64_t)(orc_splitmix64(&st) % span));
}

void orc_permutation_i64(uint64_t seed, int64_t* out, size_t n) {
  uint64_t st = seed;
  for (size_t i = 0; i < n; ++i) out[i] = (int64_t)i;
  for (size_t i = n; i > 1; --i) {
    size_t j = (size_t)(orc_splitmix64(&st) % i);
    int64_t t = out[i - 1];
    out[i - 1] = out[j];
    out[j] = t;
  }
}

/* ------------------------------------------------------------------------ */
/* Scalar conversions.                                                       */
/* ------------------------------------------------------------------------ */
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary32 -> binary16, round to nearest even, with subnormals, as the
 * `half` crate's f16::from_f32 (types.rs:237-240 -> half 2.7.1). */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFFu) {
    if (man == 0) return sign | 0x7C00u;                       /* inf */
    return sign | 0x7E00u | (uint16_t)(man >> 13);             /* quiet NaN */
  }
  int32_t e = (int32_t)exp - 127 + 15;                           /* rebias */
  if (e >= 0x1F) return sign | 0x7C00u;                          /* overflow */
  if (e <= 0) {                                                  /* subnormal/zero */
    if (e < -10) return sign;                                    /* < half of min subnormal */
    uint32_t m = man | 0x800000u;                                /* implicit bit */
    uint32_t shift = (uint32_t)(14 - e);                         /* 14..24 */
    uint32_t half_bit = 1u << (shift - 1);
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t q = m >> shift;
    if (rem > half_bit || (rem == half_bit && (q & 1u))) q += 1;
    return sign | (uint16_t)q;                                   /* may carry into exp 1 */
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1;     /* carry may reach inf */
  return sign | (uint16_t)q;
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: value = man * 2^-24, exact in f32 */
    float v = (float)man * (1.0f / 16777216.0f);
    return (sign ? -v : v);
  }
  if (exp == 0x1F) return u2f(sign | 0x7F800000u | (man << 13));
  return u2f(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void orc_f32_to_bf16_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}
void orc_bf16_to_f32_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(in[i]);
}
void orc_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
}
void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------ */
/* BlockPool -- src/memory/paged.rs:21-58                                     */
/* ------------------------------------------------------------------------ */
struct orc_block_pool {
  int64_t* free_list; /* Vec<usize>; top of stack = free_list[n_free-1] */
  int64_t n_free;
  uint32_t* ref_counts; /* Vec<u32> */
  int64_t capacity;
  int32_t quant_type;
};

orc_block_pool* orc_pool_new(int64_t capacity, int32_t quant_type) {
  /* paged.rs:28-34 */
  if (capacity < 0) return NULL;
  orc_block_pool* p = (orc_block_pool*)calloc(1, sizeof(*p));
  p->free_list = (int64_t*)malloc(sizeof(int64_t) * (size_t)(capacity ? capacity : 1));
  p->ref_counts = (uint32_t*)calloc((size_t)(capacity ? capacity : 1), sizeof(uint32_t));
  for (int64_t i = 0; i < capacity; ++i) p->free_list[i] = i;
  p->n_free = capacity;
  p->capacity = capacity;
  p->quant_type = quant_type;
  return p;
}

orc_block_pool* orc_pool_new_ordered(const int64_t* order, int64_t capacity, int32_t quant_type) {
  orc_block_pool* p = orc_pool_new(capacity, quant_type);
  if (!p) return NULL;
  for (int64_t i = 0; i < capacity; ++i) p->free_list[i] = order[i];
  return p;
}

void orc_pool_destroy(orc_block_pool* p) {
  if (!p) return;
  free(p->free_list);
  free(p->ref_counts);
  free(p);
}

int64_t orc_pool_allocate(orc_block_pool* p) {
  /* paged.rs:36-42: Vec::pop() takes the LAST element. */
  if (p->n_free == 0) return -1;
  int64_t id = p->free_list[--p->n_free];
  p->ref_counts[id] = 1;
  return id;
}

int orc_pool_share(orc_block_pool* p, int64_t id) {
  /* paged.rs:44-46.  The reference also increments a free block's count,
   * leaving it on the free list while referenced; that is rejected here. */
  if (id < 0 || id >= p->capacity || p->ref_counts[id] == 0) return ORC_INVALID_INPUT;
  p->ref_counts[id] += 1;
  return ORC_OK;
}

int orc_pool_free(orc_block_pool* p, int64_t id) {
  /* paged.rs:48-53; ref 0 would underflow the reference's u32. */
  if (id < 0 || id >= p->capacity || p->ref_counts[id] == 0) return ORC_INVALID_INPUT;
  p->ref_counts[id] -= 1;
  if (p->ref_counts[id] == 0) p->free_list[p->n_free++] = id;
  return ORC_OK;
}

int32_t orc_pool_quant_type(const orc_block_pool* p) { return p->quant_type; }
int64_t orc_pool_num_free(const orc_block_pool* p) { return p->n_free; }
int64_t orc_pool_ref_count(const orc_block_pool* p, int64_t id) {
  if (id < 0 || id >= p->capacity) return -1;
  return (int64_t)p->ref_counts[id];
}
void orc_pool_free_list(const orc_block_pool* p, int64_t* out) {
  memcpy(out, p->free_list, sizeof(int64_t) * (size_t)p->n_free);
}

/* ------------------------------------------------------------------------ */
/* Q8_0 -- src/backend/arm/quant.rs:149-183 (x86 scalar path, :265-268)     */
/* ------------------------------------------------------------------------ */
/* Rust `f as i32` saturates and maps NaN to 0. */
static int32_t rust_f32_as_i32(float f) {
  if (f != f) return 0;
  if (f >= 2147483648.0f) return INT32_MAX;
  if (f <= -2147483648.0f) return INT32_MIN;
  return (int32_t)f;
}

int orc_quantize_row_q8_0(const float* x, size_t n, uint8_t* y) {
  if (n % ORC_QK8_0) return ORC_INVALID_INPUT; /* quant.rs:150 assert */
  size_t nb = n / ORC_QK8_0;
  for (size_t i = 0; i < nb; ++i) {
    const float* xb = x + i * ORC_QK8_0;
    uint8_t* rec = y + i * ORC_BLOCK_Q8_0_BYTES;
    float amax = 0.0f; /* quant.rs:157-163: `>` ignores NaN */
    for (int j = 0; j < ORC_QK8_0; ++j) {
      float a = fabsf(xb[j]);
      if (a > amax) amax = a;
    }
    if (amax == 0.0f) { /* quant.rs:166-170 */
      memset(rec, 0, ORC_BLOCK_Q8_0_BYTES);
      continue;
    }
    float scale = amax / 127.0f; /* quant.rs:173, f32 divide */
    for (int j = 0; j < ORC_QK8_0; ++j) {
      int32_t v = rust_f32_as_i32(roundf(xb[j] / scale)); /* quant.rs:176-177 */
      if (v > 127) v = 127;
      if (v < -128) v = -128; /* quant.rs:178 */
      rec[2 + j] = (uint8_t)(int8_t)v;
    }
    uint16_t d = orc_f32_to_f16(scale); /* quant.rs:181, unrounded scale above */
    rec[0] = (uint8_t)(d & 0xFF);       /* little-endian u16, repr(C) */
    rec[1] = (uint8_t)(d >> 8);
  }
  return ORC_OK;
}

void orc_dequantize_row_q8_0(const uint8_t* y, size_t n, float* x) {
  size_t nb = n / ORC_QK8_0;
  for (size_t i = 0; i < nb; ++i) {
    const uint8_t* rec = y + i * ORC_BLOCK_Q8_0_BYTES;
    float d = orc_f16_to_f32((uint16_t)(rec[0] | (rec[1] << 8)));
    for (int j = 0; j < ORC_QK8_0; ++j) x[i * ORC_QK8_0 + j] = d * (float)(int8_t)rec[2 + j];
  }
}

/* ------------------------------------------------------------------------ */
/* Q4_0 -- block types.rs:15-22, dequantisation vec_dot.rs:425-440; the     */
/* quantiser restates ggml's quantize_row_q4_0_ref (none in the reference)  */
/* ------------------------------------------------------------------------ */
/* ggml's (int8_t)(float) as the x86 build computes it: cvttss2si truncates
 * toward zero and returns 0x80000000 (low byte 0) for NaN and out-of-range
 * values; the cast keeps the low byte.  For finite x with a finite 1/d the
 * argument x * id + 8.5 lies in [0, 16.5]; it is NaN or infinite only when
 * x or 1/d is (an infinite element, or |d| below 2^-128). */
static int32_t q4_trunc_i8(float f) {
  if (f != f || fabsf(f) >= 2147483648.0f) return 0;
  return (int32_t)(int8_t)(int32_t)f;
}

int orc_quantize_row_q4_0(const float* x, size_t n, uint8_t* y) {
  if (n % ORC_QK4_0) return ORC_INVALID_INPUT;
  size_t nb = n / ORC_QK4_0;
  for (size_t i = 0; i < nb; ++i) {
    const float* xb = x + i * ORC_QK4_0;
    uint8_t* rec = y + i * ORC_BLOCK_Q4_0_BYTES;
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < ORC_QK4_0; ++j) { /* strict <: the first of equal magnitudes; NaN never wins */
      float a = fabsf(xb[j]);
      if (amax < a) {
        amax = a;
        max = xb[j];
      }
    }
    const float d = max / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = orc_f32_to_f16(d);
    rec[0] = (uint8_t)(dh & 0xFF);
    rec[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < ORC_QK4_0 / 2; ++j) {
      int32_t q0 = q4_trunc_i8(xb[j] * id + 8.5f);
      int32_t q1 = q4_trunc_i8(xb[j + ORC_QK4_0 / 2] * id + 8.5f);
      if (q0 > 15) q0 = 15;
      if (q1 > 15) q1 = 15;
      rec[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
  }
  return ORC_OK;
}

void orc_dequantize_row_q4_0(const uint8_t* y, size_t n, float* x) {
  size_t nb = n / ORC_QK4_0;
  for (size_t i = 0; i < nb; ++i) {
    const uint8_t* rec = y + i * ORC_BLOCK_Q4_0_BYTES;
    float d = orc_f16_to_f32((uint16_t)(rec[0] | (rec[1] << 8)));
    for (int j = 0; j < ORC_QK4_0 / 2; ++j) {
      x[i * ORC_QK4_0 + j] = d * (float)((int32_t)(rec[2 + j] & 0xF) - 8);
      x[i * ORC_QK4_0 + j + ORC_QK4_0 / 2] = d * (float)((int32_t)(rec[2 + j] >> 4) - 8);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Q4_1 -- block types.rs:24-32; quantiser and dequantiser restate ggml's    */
/* (the reference has no code for Q4_1)                                     */
/* ------------------------------------------------------------------------ */
int orc_quantize_row_q4_1(const float* x, size_t n, uint8_t* y) {
  if (n % ORC_QK4_1) return ORC_INVALID_INPUT;
  size_t nb = n / ORC_QK4_1;
  for (size_t i = 0; i < nb; ++i) {
    const float* xb = x + i * ORC_QK4_1;
    uint8_t* rec = y + i * ORC_BLOCK_Q4_1_BYTES;
    float mn = FLT_MAX, mx = -FLT_MAX;
    for (int j = 0; j < ORC_QK4_1; ++j) {
      if (xb[j] < mn) mn = xb[j];
      if (xb[j] > mx) mx = xb[j];
    }
    const float d = (mx - mn) / 15.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = orc_f32_to_f16(d), mh = orc_f32_to_f16(mn);
    rec[0] = (uint8_t)(dh & 0xFF);
    rec[1] = (uint8_t)(dh >> 8);
    rec[2] = (uint8_t)(mh & 0xFF);
    rec[3] = (uint8_t)(mh >> 8);
    for (int j = 0; j < ORC_QK4_1 / 2; ++j) {
      int32_t q0 = q4_trunc_i8((xb[j] - mn) * id + 0.5f);
      int32_t q1 = q4_trunc_i8((xb[j + ORC_QK4_1 / 2] - mn) * id + 0.5f);
      if (q0 > 15) q0 = 15;
      if (q1 > 15) q1 = 15;
      rec[4 + j] = (uint8_t)(q0 | (q1 << 4));
    }
  }
  return ORC_OK;
}

void orc_dequantize_row_q4_1(const uint8_t* y, size_t n, float* x) {
  size_t nb = n / ORC_QK4_1;
  for (size_t i = 0; i < nb; ++i) {
    const uint8_t* rec = y + i * ORC_BLOCK_Q4_1_BYTES;
    float d = orc_f16_to_f32((uint16_t)(rec[0] | (rec[1] << 8)));
    float m = orc_f16_to_f32((uint16_t)(rec[2] | (rec[3] << 8)));
    for (int j = 0; j < ORC_QK4_1 / 2; ++j) {
      x[i * ORC_QK4_1 + j] = d * (float)(rec[4 + j] & 0xF) + m;
      x[i * ORC_QK4_1 + j + ORC_QK4_1 / 2] = d * (float)(rec[4 + j] >> 4) + m;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Q5_0 / Q5_1 -- ggml's quantize_row_q5_{0,1}_ref and dequantize_row_q5_*  */
/* (the reference has the type ids, types.rs:116-117, and nothing else)     */
/* ------------------------------------------------------------------------ */
/* (uint8_t)(float) on x86: the same cvttss2si, low byte kept unsigned. */
static int32_t q5_trunc_u8(float f) {
  if (f != f || fabsf(f) >= 2147483648.0f) return 0;
  return (int32_t)(uint8_t)(int32_t)f;
}

/* qh: bit e = bit 4 of element e's 5-bit value; qs as Q4's. */
static void q5_pack(const int32_t* q, uint8_t* qh4, uint8_t* qs16) {
  uint32_t qh = 0;
  for (int j = 0; j < 16; ++j) {
    qs16[j] = (uint8_t)((q[j] & 0x0F) | ((q[j + 16] & 0x0F) << 4));
    qh |= (((uint32_t)q[j] & 0x10u) >> 4) << j;
    qh |= (((uint32_t)q[j + 16] & 0x10u) >> 4) << (j + 16);
  }
  for (int b = 0; b < 4; ++b) qh4[b] = (uint8_t)(qh >> (8 * b));
}

static int32_t q5_value(const uint8_t* qh4, const uint8_t* qs16, int e) {
  uint32_t qh = (uint32_t)qh4[0] | ((uint32_t)qh4[1] << 8) | ((uint32_t)qh4[2] << 16) | ((uint32_t)qh4[3] << 24);
  int32_t nib = e < 16 ? (qs16[e] & 0xF) : (qs16[e - 16] >> 4);
  return nib | (int32_t)(((qh >> e) & 1u) << 4);
}

int orc_quantize_row_q5_0(const float* x, size_t n, uint8_t* y) {
  if (n % ORC_QK5_0) return ORC_INVALID_INPUT;
  for (size_t i = 0; i < n / ORC_QK5_0; ++i) {
    const float* xb = x + i * ORC_QK5_0;
    uint8_t* rec = y + i * ORC_BLOCK_Q5_0_BYTES;
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < ORC_QK5_0; ++j) { /* strict <: the first of equal magnitudes; NaN never wins */
      float a = fabsf(xb[j]);
      if (amax < a) {
        amax = a;
        max = xb[j];
      }
    }
    const float d = max / -16.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = orc_f32_to_f16(d);
    rec[0] = (uint8_t)(dh & 0xFF);
    rec[1] = (uint8_t)(dh >> 8);
    int32_t q[ORC_QK5_0];
    for (int j = 0; j < ORC_QK5_0; ++j) {
      int32_t v = q4_trunc_i8(xb[j] * id + 16.5f);
      q[j] = v > 31 ? 31 : v;
    }
    q5_pack(q, rec + 2, rec + 6);
  }
  return ORC_OK;
}

void orc_dequantize_row_q5_0(const uint8_t* y, size_t n, float* x) {
  for (size_t i = 0; i < n / ORC_QK5_0; ++i) {
    const uint8_t* rec = y + i * ORC_BLOCK_Q5_0_BYTES;
    float d = orc_f16_to_f32((uint16_t)(rec[0] | (rec[1] << 8)));
    for (int e = 0; e < ORC_QK5_0; ++e) x[i * ORC_QK5_0 + e] = d * (float)(q5_value(rec + 2, rec + 6, e) - 16);
  }
}

int orc_quantize_row_q5_1(const float* x, size_t n, uint8_t* y) {
  if (n % ORC_QK5_1) return ORC_INVALID_INPUT;
  for (size_t i = 0; i < n / ORC_QK5_1; ++i) {
    const float* xb = x + i * ORC_QK5_1;
    uint8_t* rec = y + i * ORC_BLOCK_Q5_1_BYTES;
    float mn = FLT_MAX, mx = -FLT_MAX;
    for (int j = 0; j < ORC_QK5_1; ++j) {
      if (xb[j] < mn) mn = xb[j];
      if (xb[j] > mx) mx = xb[j];
    }
    const float d = (mx - mn) / 31.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = orc_f32_to_f16(d), mh = orc_f32_to_f16(mn);
    rec[0] = (uint8_t)(dh & 0xFF);
    rec[1] = (uint8_t)(dh >> 8);
    rec[2] = (uint8_t)(mh & 0xFF);
    rec[3] = (uint8_t)(mh >> 8);
    int32_t q[ORC_QK5_1];
    for (int j = 0; j < ORC_QK5_1; ++j) q[j] = q5_trunc_u8((xb[j] - mn) * id + 0.5f);
    q5_pack(q, rec + 4, rec + 8);
  }
  return ORC_OK;
}

void orc_dequantize_row_q5_1(const uint8_t* y, size_t n, float* x) {
  for (size_t i = 0; i < n / ORC_QK5_1; ++i) {
    const uint8_t* rec = y + i * ORC_BLOCK_Q5_1_BYTES;
    float d = orc_f16_to_f32((uint16_t)(rec[0] | (rec[1] << 8)));
    float m = orc_f16_to_f32((uint16_t)(rec[2] | (rec[3] << 8)));
    for (int e = 0; e < ORC_QK5_1; ++e) x[i * ORC_QK5_1 + e] = d * (float)q5_value(rec + 4, rec + 8, e) + m;
  }
}

/* ------------------------------------------------------------------------ */
/* rope_f32 -- src/backend/arm/rope.rs:6-44                                   */
/* ------------------------------------------------------------------------ */
int orc_rope_f32(const float* x, float* out, size_t n, int64_t pos, int32_t n_dims, int32_t head_dim,
                 float freq_base) {
  if (head_dim <= 0 || n % (size_t)head_dim || n_dims % 2 || n_dims < 0 || n_dims > head_dim)
    return ORC_INVALID_INPUT; /* rope.rs:15-16 asserts; n_dims <= head_dim as forward.rs calls it */
  memcpy(out, x, n * sizeof(float)); /* rope.rs:18 */
  size_t n_heads = n / (size_t)head_dim;
  for (size_t h = 0; h < n_heads; ++h) {
    size_t offset = h * (size_t)head_dim;
    for (int32_t i = 0; i < n_dims; i += 2) { /* rope.rs:25 */
      size_t idx = offset + (size_t)i;
      if (idx + 1 >= n) break; /* rope.rs:27-29 */
      float dim = (float)i;
      /* rope.rs:31: `pos as f32 * freq_base.powf(-dim / n_dims as f32)` */
      float theta = (float)pos * powf(freq_base, -dim / (float)n_dims);
      float cos_theta = cosf(theta), sin_theta = sinf(theta);
      float x0 = x[idx], x1 = x[idx + 1];
      out[idx] = x0 * cos_theta - x1 * sin_theta; /* rope.rs:38-39, two roundings then one */
      out[idx + 1] = x0 * sin_theta + x1 * cos_theta;
    }
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* flash_attn_f32 -- src/backend/arm/flash_attn.rs:6-72                       */
/* ------------------------------------------------------------------------ */
void orc_flash_attn_f32(const float* q, const float* k, const float* v, const float* mask,
                        float* out, int32_t head_dim, int32_t n_kv, float scale) {
  for (int32_t i = 0; i < head_dim; ++i) out[i] = 0.0f; /* :21-23 */
  float m = -INFINITY, s = 0.0f;                         /* :25-26 */
  for (int32_t i_kv = 0; i_kv < n_kv; ++i_kv) {          /* :28 */
    float kq = 0.0f;
    const float* kr = k + (size_t)i_kv * head_dim;
    for (int32_t d = 0; d < head_dim; ++d) kq += q[d] * kr[d]; /* :29-32 sequential */
    kq *= scale;                                               /* :33 */
    if (mask) {                                                /* :35-40 */
      kq += mask[i_kv];
      if (mask[i_kv] == -INFINITY) continue;
    }
    float m_old = m, k_vs, m_scale;
    if (kq > m) { /* :46-53 */
      m = kq;
      m_scale = expf(m_old - m);
      k_vs = 1.0f;
    } else {
      m_scale = 1.0f;
      k_vs = expf(kq - m);
    }
    const float* vr = v + (size_t)i_kv * head_dim;
    for (int32_t d = 0; d < head_dim; ++d) out[d] *= m_scale;     /* :55-57 */
    for (int32_t d = 0; d < head_dim; ++d) out[d] += vr[d] * k_vs; /* :59-61 */
    s = s * m_scale + k_vs;                                         /* :63 */
  }
  if (s > 0.0f) { /* :66-71 */
    float inv_s = 1.0f / s;
    for (int32_t d = 0; d < head_dim; ++d) out[d] *= inv_s;
  }
}

int orc_backend_flash_attention(const float* q, const float* k, const float* v,
                                const float* mask, float* out, int32_t n_heads,
                                int32_t head_dim, int32_t n_kv) {
  /* src/backend/arm.rs:304-370: every head reads the same K/V and mask. */
  if (n_heads <= 0 || head_dim <= 0 || n_kv < 0) return ORC_INVALID_INPUT;
  float scale = 1.0f / sqrtf((float)head_dim);
  for (int32_t h = 0; h < n_heads; ++h)
    orc_flash_attn_f32(q + (size_t)h * head_dim, k, v, mask, out + (size_t)h * head_dim,
                       head_dim, n_kv, scale);
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* Paged cache restatement.                                                  */
/* ------------------------------------------------------------------------ */
static size_t elem_bytes(int32_t dtype) {
  switch (dtype) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    case ORC_BF16: return 2;
    default: return 0;
  }
}

static int desc_ok(const orc_cache_desc* c) {
  if (c->num_blocks <= 0 || c->block_size <= 0 || c->n_kv_heads <= 0 || c->head_dim <= 0) return 0;
  if (c->dtype == ORC_Q8_0) return c->head_dim % ORC_QK8_0 == 0;
  if (c->dtype == ORC_Q4_0) return c->head_dim % ORC_QK4_0 == 0;
  if (c->dtype == ORC_Q4_1) return c->head_dim % ORC_QK4_1 == 0;
  if (c->dtype == ORC_Q5_0 || c->dtype == ORC_Q5_1) return c->head_dim % 32 == 0;
  return elem_bytes(c->dtype) != 0;
}

size_t orc_page_bytes(const orc_cache_desc* c) {
  size_t bs = (size_t)c->block_size, d = (size_t)c->head_dim;
  if (c->dtype == ORC_Q8_0) return bs * d + bs * (d / ORC_QK8_0) * 2;
  if (c->dtype == ORC_Q4_0) return bs * (d / 2) + bs * (d / ORC_QK4_0) * 2;
  if (c->dtype == ORC_Q4_1) return bs * (d / 2) + bs * (d / ORC_QK4_1) * 4;
  if (c->dtype == ORC_Q5_0) return bs * (d / 2) + bs * (d / ORC_QK5_0) * 6;
  if (c->dtype == ORC_Q5_1) return bs * (d / 2) + bs * (d / ORC_QK5_1) * 8;
  return bs * d * elem_bytes(c->dtype);
}

/* Q5 pages: the nibble plane [block_size][d / 2], then per token a side row
 * of d/32 qh words and d/32 metadata words (fp16 d, or the (d, m) pair).
 * A ggml record is {meta, qh, qs}. */
static int is_q5(int32_t dt) { return dt == ORC_Q5_0 || dt == ORC_Q5_1; }
static size_t q5_meta_bytes(int32_t dt) { return dt == ORC_Q5_1 ? 4 : 2; }
static size_t q5_record_bytes(int32_t dt) { return dt == ORC_Q5_1 ? ORC_BLOCK_Q5_1_BYTES : ORC_BLOCK_Q5_0_BYTES; }

static void q5_put_row(const orc_cache_desc* c, uint8_t* page, int32_t slot, const float* x) {
  size_t d = (size_t)c->head_dim, ng = d / 32, mb = q5_meta_bytes(c->dtype);
  uint8_t rec[ORC_BLOCK_Q5_1_BYTES];
  uint8_t* qs = page + (size_t)slot * (d / 2);
  uint8_t* side = page + (size_t)c->block_size * (d / 2) + (size_t)slot * ng * (4 + mb);
  for (size_t g = 0; g < ng; ++g) {
    if (c->dtype == ORC_Q5_1) orc_quantize_row_q5_1(x + g * 32, 32, rec);
    else orc_quantize_row_q5_0(x + g * 32, 32, rec);
    memcpy(side + ng * 4 + g * mb, rec, mb);
    memcpy(side + g * 4, rec + mb, 4);
    memcpy(qs + g * 16, rec + mb + 4, 16);
  }
}

static void q5_get_row(const orc_cache_desc* c, const uint8_t* page, int32_t slot, uint8_t* dst) {
  size_t d = (size_t)c->head_dim, ng = d / 32, mb = q5_meta_bytes(c->dtype), rb = q5_record_bytes(c->dtype);
  const uint8_t* qs = page + (size_t)slot * (d / 2);
  const uint8_t* side = page + (size_t)c->block_size * (d / 2) + (size_t)slot * ng * (4 + mb);
  for (size_t g = 0; g < ng; ++g) {
    uint8_t* rec = dst + g * rb;
    memcpy(rec, side + ng * 4 + g * mb, mb);
    memcpy(rec + mb, side + g * 4, 4);
    memcpy(rec + mb + 4, qs + g * 16, 16);
  }
}

static uint8_t* page_ptr(const orc_cache_desc* c, const uint8_t* pool, int64_t block, int32_t h) {
  return (uint8_t*)pool + ((size_t)block * (size_t)c->n_kv_heads + (size_t)h) * orc_page_bytes(c);
}

/* Write one token row (head_dim values) of one head into its page slot. */
static void put_row(const orc_cache_desc* c, uint8_t* page, int32_t slot, const void* src_row) {
  size_t d = (size_t)c->head_dim;
  if (is_q5(c->dtype)) {
    q5_put_row(c, page, slot, (const float*)src_row);
  } else if (c->dtype == ORC_Q8_0) {
    size_t ng = d / ORC_QK8_0;
    uint8_t rec[ORC_BLOCK_Q8_0_BYTES];
    uint8_t* qs = page + (size_t)slot * d;
    uint8_t* sc = page + (size_t)c->block_size * d + (size_t)slot * ng * 2;
    for (size_t g = 0; g < ng; ++g) {
      orc_quantize_row_q8_0((const float*)src_row + g * ORC_QK8_0, ORC_QK8_0, rec);
      memcpy(qs + g * ORC_QK8_0, rec + 2, ORC_QK8_0);
      sc[g * 2] = rec[0];
      sc[g * 2 + 1] = rec[1];
    }
  } else if (c->dtype == ORC_Q4_1) {
    /* qs plane [block_size][d / 2], then [block_size][d / 32] (d, m) fp16 pairs. */
    size_t ng = d / ORC_QK4_1;
    uint8_t rec[ORC_BLOCK_Q4_1_BYTES];
    uint8_t* qs = page + (size_t)slot * (d / 2);
    uint8_t* sc = page + (size_t)c->block_size * (d / 2) + (size_t)slot * ng * 4;
    for (size_t g = 0; g < ng; ++g) {
      orc_quantize_row_q4_1((const float*)src_row + g * ORC_QK4_1, ORC_QK4_1, rec);
      memcpy(qs + g * 16, rec + 4, 16);
      memcpy(sc + g * 4, rec, 4);
    }
  } else if (c->dtype == ORC_Q4_0) {
    /* qs plane [block_size][d / 2] (each group's 16 bytes as in the block),
     * then the d plane [block_size][d / 32] fp16. */
    size_t ng = d / ORC_QK4_0;
    uint8_t rec[ORC_BLOCK_Q4_0_BYTES];
    uint8_t* qs = page + (size_t)slot * (d / 2);
    uint8_t* sc = page + (size_t)c->block_size * (d / 2) + (size_t)slot * ng * 2;
    for (size_t g = 0; g < ng; ++g) {
      orc_quantize_row_q4_0((const float*)src_row + g * ORC_QK4_0, ORC_QK4_0, rec);
      memcpy(qs + g * 16, rec + 2, 16);
      sc[g * 2] = rec[0];
      sc[g * 2 + 1] = rec[1];
    }
  } else {
    size_t rb = d * elem_bytes(c->dtype);
    memcpy(page + (size_t)slot * rb, src_row, rb);
  }
}

int orc_kv_append(const orc_cache_desc* c, uint8_t* k_pool, uint8_t* v_pool,
                  const void* k, const void* v, const int64_t* slots, int32_t n_tokens) {
  if (!desc_ok(c) || n_tokens < 0) return ORC_INVALID_INPUT;
  size_t src_eb = (c->dtype == ORC_Q8_0 || c->dtype == ORC_Q4_0 || c->dtype == ORC_Q4_1 || is_q5(c->dtype))
                      ? 4
                      : elem_bytes(c->dtype);
  size_t row = (size_t)c->head_dim * src_eb;
  int64_t n_slots = c->num_blocks * c->block_size;
  for (int32_t t = 0; t < n_tokens; ++t) {
    int64_t slot = slots[t];
    if (slot < 0) continue; /* padding token */
    if (slot >= n_slots) return ORC_INVALID_INPUT;
    int64_t blk = slot / c->block_size;
    int32_t off = (int32_t)(slot % c->block_size);
    for (int32_t h = 0; h < c->n_kv_heads; ++h) {
      size_t src_off = ((size_t)t * c->n_kv_heads + h) * row;
      put_row(c, page_ptr(c, k_pool, blk, h), off, (const uint8_t*)k + src_off);
      put_row(c, page_ptr(c, v_pool, blk, h), off, (const uint8_t*)v + src_off);
    }
  }
  return ORC_OK;
}

/* Copy the stored row of `slot` in a page: native bytes, or a BlockQ8_0 AoS
 * record sequence for Q8_0. */
static void get_row_raw(const orc_cache_desc* c, const uint8_t* page, int32_t slot, uint8_t* dst) {
  size_t d = (size_t)c->head_dim;
  if (is_q5(c->dtype)) {
    q5_get_row(c, page, slot, dst);
  } else if (c->dtype == ORC_Q8_0) {
    size_t ng = d / ORC_QK8_0;
    const uint8_t* qs = page + (size_t)slot * d;
    const uint8_t* sc = page + (size_t)c->block_size * d + (size_t)slot * ng * 2;
    for (size_t g = 0; g < ng; ++g) {
      uint8_t* rec = dst + g * ORC_BLOCK_Q8_0_BYTES;
      rec[0] = sc[g * 2];
      rec[1] = sc[g * 2 + 1];
      memcpy(rec + 2, qs + g * ORC_QK8_0, ORC_QK8_0);
    }
  } else if (c->dtype == ORC_Q4_1) {
    size_t ng = d / ORC_QK4_1;
    const uint8_t* qs = page + (size_t)slot * (d / 2);
    const uint8_t* sc = page + (size_t)c->block_size * (d / 2) + (size_t)slot * ng * 4;
    for (size_t g = 0; g < ng; ++g) {
      uint8_t* rec = dst + g * ORC_BLOCK_Q4_1_BYTES;
      memcpy(rec, sc + g * 4, 4);
      memcpy(rec + 4, qs + g * 16, 16);
    }
  } else if (c->dtype == ORC_Q4_0) {
    size_t ng = d / ORC_QK4_0;
    const uint8_t* qs = page + (size_t)slot * (d / 2);
    const uint8_t* sc = page + (size_t)c->block_size * (d / 2) + (size_t)slot * ng * 2;
    for (size_t g = 0; g < ng; ++g) {
      uint8_t* rec = dst + g * ORC_BLOCK_Q4_0_BYTES;
      rec[0] = sc[g * 2];
      rec[1] = sc[g * 2 + 1];
      memcpy(rec + 2, qs + g * 16, 16);
    }
  } else {
    size_t rb = d * elem_bytes(c->dtype);
    memcpy(dst, page + (size_t)slot * rb, rb);
  }
}

static size_t row_out_bytes(const orc_cache_desc* c) {
  if (c->dtype == ORC_Q8_0) return (size_t)(c->head_dim / ORC_QK8_0) * ORC_BLOCK_Q8_0_BYTES;
  if (c->dtype == ORC_Q4_0) return (size_t)(c->head_dim / ORC_QK4_0) * ORC_BLOCK_Q4_0_BYTES;
  if (c->dtype == ORC_Q4_1) return (size_t)(c->head_dim / ORC_QK4_1) * ORC_BLOCK_Q4_1_BYTES;
  if (is_q5(c->dtype)) return (size_t)(c->head_dim / 32) * q5_record_bytes(c->dtype);
  return (size_t)c->head_dim * elem_bytes(c->dtype);
}

/* Widen one stored row to f32 (bf16/f16 exact, Q8_0 = f32(d)*q, Q4_0 =
 * f32(d)*(nibble-8)). */
static void get_row_f32(const orc_cache_desc* c, const uint8_t* page, int32_t slot, float* dst) {
  size_t d = (size_t)c->head_dim;
  switch (c->dtype) {
    case ORC_F32: memcpy(dst, page + (size_t)slot * d * 4, d * 4); break;
    case ORC_BF16: orc_bf16_to_f32_array((const uint16_t*)(page + (size_t)slot * d * 2), dst, d); break;
    case ORC_F16: orc_f16_to_f32_array((const uint16_t*)(page + (size_t)slot * d * 2), dst, d); break;
    case ORC_Q8_0: {
      uint8_t rec[8 * ORC_BLOCK_Q8_0_BYTES * 4];
      size_t ng = d / ORC_QK8_0;
      uint8_t* buf = ng * ORC_BLOCK_Q8_0_BYTES <= sizeof(rec) ? rec : (uint8_t*)malloc(ng * ORC_BLOCK_Q8_0_BYTES);
      get_row_raw(c, page, slot, buf);
      orc_dequantize_row_q8_0(buf, d, dst);
      if (buf != rec) free(buf);
      break;
    }
    case ORC_Q4_1: {
      uint8_t rec[8 * ORC_BLOCK_Q4_1_BYTES * 4];
      size_t ng = d / ORC_QK4_1;
      uint8_t* buf = ng * ORC_BLOCK_Q4_1_BYTES <= sizeof(rec) ? rec : (uint8_t*)malloc(ng * ORC_BLOCK_Q4_1_BYTES);
      get_row_raw(c, page, slot, buf);
      orc_dequantize_row_q4_1(buf, d, dst);
      if (buf != rec) free(buf);
      break;
    }
    case ORC_Q5_0:
    case ORC_Q5_1: {
      uint8_t rec[8 * ORC_BLOCK_Q5_1_BYTES * 4];
      size_t nb = (d / 32) * q5_record_bytes(c->dtype);
      uint8_t* buf = nb <= sizeof(rec) ? rec : (uint8_t*)malloc(nb);
      get_row_raw(c, page, slot, buf);
      if (c->dtype == ORC_Q5_1) orc_dequantize_row_q5_1(buf, d, dst);
      else orc_dequantize_row_q5_0(buf, d, dst);
      if (buf != rec) free(buf);
      break;
    }
    case ORC_Q4_0: {
      uint8_t rec[8 * ORC_BLOCK_Q4_0_BYTES * 4];
      size_t ng = d / ORC_QK4_0;
      uint8_t* buf = ng * ORC_BLOCK_Q4_0_BYTES <= sizeof(rec) ? rec : (uint8_t*)malloc(ng * ORC_BLOCK_Q4_0_BYTES);
      get_row_raw(c, page, slot, buf);
      orc_dequantize_row_q4_0(buf, d, dst);
      if (buf != rec) free(buf);
      break;
    }
  }
}

int orc_kv_gather(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                  const int32_t* block_tables, int32_t max_blocks, const int32_t* ctx_lens,
                  const int32_t* start_pos, const int64_t* cu_out, int32_t n_seqs,
                  void* k_out, void* v_out) {
  if (!desc_ok(c) || n_seqs < 0) return ORC_INVALID_INPUT;
  size_t rb = row_out_bytes(c);
  for (int32_t b = 0; b < n_seqs; ++b) {
    int32_t st = start_pos ? start_pos[b] : 0;
    int32_t n = ctx_lens[b] - st;
    if (st < 0 || n < 0) return ORC_INVALID_INPUT;
    for (int32_t h = 0; h < c->n_kv_heads; ++h)
      for (int32_t i = 0; i < n; ++i) {
        int32_t pos = st + i;
        int32_t lb = pos / c->block_size;
        if (lb >= max_blocks) return ORC_INVALID_INPUT;
        int32_t blk = block_tables[(size_t)b * max_blocks + lb];
        if (blk < 0 || blk >= c->num_blocks) return ORC_INVALID_INPUT;
        size_t o = (((size_t)cu_out[b] * c->n_kv_heads) + (size_t)h * n + i) * rb;
        get_row_raw(c, page_ptr(c, k_pool, blk, h), pos % c->block_size, (uint8_t*)k_out + o);
        get_row_raw(c, page_ptr(c, v_pool, blk, h), pos % c->block_size, (uint8_t*)v_out + o);
      }
  }
  return ORC_OK;
}

int orc_kv_evict(const orc_cache_desc* c, uint8_t* k_pool, uint8_t* v_pool,
                 const int32_t* blocks, int32_t n) {
  if (!desc_ok(c) || n < 0) return ORC_INVALID_INPUT;
  size_t pb = orc_page_bytes(c) * (size_t)c->n_kv_heads;
  for (int32_t i = 0; i < n; ++i) {
    if (blocks[i] < 0 || blocks[i] >= c->num_blocks) return ORC_INVALID_INPUT;
    memset(k_pool + (size_t)blocks[i] * pb, 0, pb);
    memset(v_pool + (size_t)blocks[i] * pb, 0, pb);
  }
  return ORC_OK;
}

/* Widen keys/values [st, st+n) of kv head h of sequence b to f32 rows. */
static int widen_seq(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                     const int32_t* table, int32_t max_blocks, int32_t h, int32_t st, int32_t n,
                     float* kf, float* vf) {
  for (int32_t i = 0; i < n; ++i) {
    int32_t pos = st + i, lb = pos / c->block_size;
    if (lb >= max_blocks) return ORC_INVALID_INPUT;
    int32_t blk = table[lb];
    if (blk < 0 || blk >= c->num_blocks) return ORC_INVALID_INPUT;
    get_row_f32(c, page_ptr(c, k_pool, blk, h), pos % c->block_size, kf + (size_t)i * c->head_dim);
    get_row_f32(c, page_ptr(c, v_pool, blk, h), pos % c->block_size, vf + (size_t)i * c->head_dim);
  }
  return ORC_OK;
}

int orc_paged_decode(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                     const float* q, int32_t n_heads, const int32_t* block_tables,
                     int32_t max_blocks, const int32_t* ctx_lens, const int32_t* start_pos,
                     int32_t n_seqs, float scale, float* out) {
  if (!desc_ok(c) || n_heads <= 0 || n_heads % c->n_kv_heads) return ORC_INVALID_INPUT;
  const int32_t D = c->head_dim, Hkv = c->n_kv_heads;
  for (int32_t b = 0; b < n_seqs; ++b) {
    int32_t st = start_pos ? start_pos[b] : 0;
    int32_t n = ctx_lens[b] - st;
    if (st < 0 || n < 0) return ORC_INVALID_INPUT;
    float* kf = (float*)malloc(sizeof(float) * (size_t)(n ? n : 1) * D);
    float* vf = (float*)malloc(sizeof(float) * (size_t)(n ? n : 1) * D);
    for (int32_t kvh = 0; kvh < Hkv; ++kvh) {
      int rc = widen_seq(c, k_pool, v_pool, block_tables + (size_t)b * max_blocks, max_blocks,
                         kvh, st, n, kf, vf);
      if (rc) { free(kf); free(vf); return rc; }
      for (int32_t h = 0; h < n_heads; ++h) {
        if (h * Hkv / n_heads != kvh) continue; /* forward.rs:234 GQA map */
        size_t qo = ((size_t)b * n_heads + h) * D;
        orc_flash_attn_f32(q + qo, kf, vf, NULL, out + qo, D, n, scale);
      }
    }
    free(kf);
    free(vf);
  }
  return ORC_OK;
}

int orc_paged_decode_mt(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                        const float* q, int32_t n_heads, const int32_t* block_tables,
                        int32_t max_blocks, const int32_t* ctx_lens, const int32_t* start_pos,
                        int32_t n_seqs, float scale, float* out, int32_t n_threads) {
  if (!desc_ok(c) || n_heads <= 0 || n_heads % c->n_kv_heads || n_threads <= 0) return ORC_INVALID_INPUT;
  const int32_t D = c->head_dim, Hkv = c->n_kv_heads;
  for (int32_t b = 0; b < n_seqs; ++b) {
    int32_t st = start_pos ? start_pos[b] : 0;
    if (st < 0 || ctx_lens[b] - st < 0) return ORC_INVALID_INPUT;
  }
  int bad = 0;
  const int64_t units = (int64_t)n_seqs * Hkv;
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads) reduction(| : bad)
  for (int64_t u = 0; u < units; ++u) {
    const int32_t b = (int32_t)(u / Hkv), kvh = (int32_t)(u % Hkv);
    const int32_t st = start_pos ? start_pos[b] : 0;
    const int32_t n = ctx_lens[b] - st;
    float* kf = (float*)malloc(sizeof(float) * (size_t)(n ? n : 1) * D);
    float* vf = (float*)malloc(sizeof(float) * (size_t)(n ? n : 1) * D);
    if (widen_seq(c, k_pool, v_pool, block_tables + (size_t)b * max_blocks, max_blocks, kvh, st, n, kf, vf)) {
      bad = 1;
    } else {
      for (int32_t h = 0; h < n_heads; ++h) {
        if (h * Hkv / n_heads != kvh) continue; /* forward.rs:234 GQA map */
        size_t qo = ((size_t)b * n_heads + h) * D;
        orc_flash_attn_f32(q + qo, kf, vf, NULL, out + qo, D, n, scale);
      }
    }
    free(kf);
    free(vf);
  }
  return bad ? ORC_INVALID_INPUT : ORC_OK;
}

int orc_paged_prefill_rows(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                           const float* q, int32_t n_heads, const int32_t* cu_q,
                           const int32_t* block_tables, int32_t max_blocks,
                           const int32_t* ctx_lens, int32_t b, int32_t row_begin,
                           int32_t row_end, float scale, int32_t causal, float* out) {
  if (!desc_ok(c) || n_heads <= 0 || n_heads % c->n_kv_heads) return ORC_INVALID_INPUT;
  const int32_t D = c->head_dim, Hkv = c->n_kv_heads;
  int32_t ql = cu_q[b + 1] - cu_q[b];
  int32_t ctx = ctx_lens[b];
  if (ql < 0 || ql > ctx) return ORC_INVALID_INPUT;
  float* kf = (float*)malloc(sizeof(float) * (size_t)(ctx ? ctx : 1) * D);
  float* vf = (float*)malloc(sizeof(float) * (size_t)(ctx ? ctx : 1) * D);
  for (int32_t kvh = 0; kvh < Hkv; ++kvh) {
    int rc = widen_seq(c, k_pool, v_pool, block_tables + (size_t)b * max_blocks, max_blocks, kvh,
                       0, ctx, kf, vf);
    if (rc) { free(kf); free(vf); return rc; }
    for (int32_t i = row_begin; i < row_end; ++i) {
      int32_t n_kv = causal ? (ctx - ql + i + 1) : ctx; /* causal prefix of the chunk row */
      for (int32_t h = 0; h < n_heads; ++h) {
        if (h * Hkv / n_heads != kvh) continue;
        size_t qo = ((size_t)(cu_q[b] + i) * n_heads + h) * D;
        orc_flash_attn_f32(q + qo, kf, vf, NULL, out + qo, D, n_kv, scale);
      }
    }
  }
  free(kf);
  free(vf);
  return ORC_OK;
}

int orc_paged_prefill_rows_mt(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                              const float* q, int32_t n_heads, const int32_t* cu_q,
                              const int32_t* block_tables, int32_t max_blocks,
                              const int32_t* ctx_lens, int32_t b, int32_t row_begin,
                              int32_t row_end, float scale, int32_t causal, float* out,
                              int32_t n_threads) {
  if (!desc_ok(c) || n_heads <= 0 || n_heads % c->n_kv_heads || n_threads <= 0) return ORC_INVALID_INPUT;
  const int32_t D = c->head_dim, Hkv = c->n_kv_heads;
  int32_t ql = cu_q[b + 1] - cu_q[b];
  int32_t ctx = ctx_lens[b];
  if (ql < 0 || ql > ctx) return ORC_INVALID_INPUT;
  float* kf = (float*)malloc(sizeof(float) * (size_t)(ctx ? ctx : 1) * D);
  float* vf = (float*)malloc(sizeof(float) * (size_t)(ctx ? ctx : 1) * D);
  for (int32_t kvh = 0; kvh < Hkv; ++kvh) {
    int rc = widen_seq(c, k_pool, v_pool, block_tables + (size_t)b * max_blocks, max_blocks, kvh,
                       0, ctx, kf, vf);
    if (rc) { free(kf); free(vf); return rc; }
#pragma omp parallel for schedule(dynamic, 4) num_threads(n_threads)
    for (int32_t i = row_begin; i < row_end; ++i) {
      int32_t n_kv = causal ? (ctx - ql + i + 1) : ctx; /* causal prefix of the chunk row */
      for (int32_t h = 0; h < n_heads; ++h) {
        if (h * Hkv / n_heads != kvh) continue;
        size_t qo = ((size_t)(cu_q[b] + i) * n_heads + h) * D;
        orc_flash_attn_f32(q + qo, kf, vf, NULL, out + qo, D, n_kv, scale);
      }
    }
  }
  free(kf);
  free(vf);
  return ORC_OK;
}

int orc_paged_prefill(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                      const float* q, int32_t n_heads, const int32_t* cu_q,
                      const int32_t* block_tables, int32_t max_blocks, const int32_t* ctx_lens,
                      int32_t n_seqs, float scale, int32_t causal, float* out) {
  for (int32_t b = 0; b < n_seqs; ++b) {
    int rc = orc_paged_prefill_rows(c, k_pool, v_pool, q, n_heads, cu_q, block_tables, max_blocks,
                                    ctx_lens, b, 0, cu_q[b + 1] - cu_q[b], scale, causal, out);
    if (rc) return rc;
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* Sequence / window manager over BlockPool.                                 */
/* ------------------------------------------------------------------------ */
struct orc_kv_manager {
  orc_block_pool* pool;
  int32_t bs, max_seqs, max_blocks, window;
  int32_t* table;     /* [max_seqs][max_blocks], -1 = not held */
  int64_t* pos;       /* next position (= ctx len) */
  int64_t* first;     /* lowest logical block still held */
};

orc_kv_manager* orc_mgr_new(orc_block_pool* pool, int32_t block_size, int32_t max_seqs,
                            int32_t max_blocks_per_seq, int32_t window) {
  if (!pool || block_size <= 0 || max_seqs <= 0 || max_blocks_per_seq <= 0 || window < 0) return NULL;
  orc_kv_manager* m = (orc_kv_manager*)calloc(1, sizeof(*m));
  m->pool = pool;
  m->bs = block_size;
  m->max_seqs = max_seqs;
  m->max_blocks = max_blocks_per_seq;
  m->window = window;
  m->table = (int32_t*)malloc(sizeof(int32_t) * (size_t)max_seqs * max_blocks_per_seq);
  for (size_t i = 0; i < (size_t)max_seqs * max_blocks_per_seq; ++i) m->table[i] = -1;
  m->pos = (int64_t*)calloc((size_t)max_seqs, sizeof(int64_t));
  m->first = (int64_t*)calloc((size_t)max_seqs, sizeof(int64_t));
  return m;
}

void orc_mgr_destroy(orc_kv_manager* m) {
  if (!m) return;
  free(m->table);
  free(m->pos);
  free(m->first);
  free(m);
}

int orc_mgr_seed_seq(orc_kv_manager* m, int32_t s, int64_t pos, int64_t first_block,
                     const int32_t* blocks, int32_t n) {
  if (s < 0 || s >= m->max_seqs || first_block < 0 || first_block + n > m->max_blocks) return ORC_INVALID_INPUT;
  int32_t* row = m->table + (size_t)s * m->max_blocks;
  for (int32_t j = 0; j < m->max_blocks; ++j) row[j] = -1;
  for (int32_t j = 0; j < n; ++j) row[first_block + j] = blocks[j];
  m->pos[s] = pos;
  m->first[s] = first_block;
  return ORC_OK;
}

/* One step's rules (restated on BlockPool, paged.rs:21-58):
 *  - window: before position p, every held block whose last position is
 *    < p - W + 1 drops this sequence's reference (BlockPool::free), oldest
 *    first;
 *  - a block whose refcount reaches 0 is returned to the pool's free list
 *    when the step ends, in free order (so within one step no block is
 *    freed and handed out again), and is listed in evicted_out; a block a
 *    forked sequence still holds is not;
 *  - tokens of the step written into a block the step returns get slot -1
 *    (dead: the window dropped them before the step ended). */
static int64_t mgr_drop_ref(orc_block_pool* p, int64_t id) {
  if (id < 0 || id >= p->capacity || p->ref_counts[id] == 0) return -1;
  p->ref_counts[id] -= 1; /* the push of a block reaching 0 waits for the step's end */
  return p->ref_counts[id];
}

static int mgr_end_step(orc_kv_manager* m, const int32_t* freed, int32_t n_freed, int rc) {
  for (int32_t i = 0; i < n_freed; ++i) m->pool->free_list[m->pool->n_free++] = freed[i];
  return rc;
}

int orc_mgr_append_cow(orc_kv_manager* m, const int32_t* seqs, const int32_t* n_tokens, int32_t n,
                       int32_t cow, int64_t* slots_out, int32_t* evicted_out, int32_t evicted_cap,
                       int32_t* n_evicted, int32_t* cow_src, int32_t* cow_dst, int32_t cow_cap,
                       int32_t* n_cow) {
  int32_t ne = 0, nc = 0;
  size_t t = 0;
  for (int32_t i = 0; i < n; ++i) {
    int32_t s = seqs[i];
    if (s < 0 || s >= m->max_seqs || n_tokens[i] < 0) return mgr_end_step(m, evicted_out, ne, ORC_INVALID_INPUT);
    int32_t* row = m->table + (size_t)s * m->max_blocks;
    for (int32_t k = 0; k < n_tokens[i]; ++k) {
      int64_t p = m->pos[s];
      while (m->window > 0 && m->first[s] * m->bs + m->bs - 1 < p - m->window + 1) {
        int64_t j = m->first[s];
        if (j >= m->max_blocks) return mgr_end_step(m, evicted_out, ne, ORC_INVALID_INPUT);
        if (row[j] >= 0) {
          int32_t id = row[j];
          int64_t left = mgr_drop_ref(m->pool, id);
          if (left < 0) return mgr_end_step(m, evicted_out, ne, ORC_INVALID_INPUT);
          if (left == 0) {
            if (ne >= evicted_cap) { /* undo: the block stays free */
              m->pool->free_list[m->pool->n_free++] = id;
              return mgr_end_step(m, evicted_out, ne, ORC_INVALID_INPUT);
            }
            evicted_out[ne++] = id;
            /* Dead tokens: every slot of this step inside the block. */
            for (size_t u = 0; u < t; ++u)
              if (slots_out[u] >= 0 && slots_out[u] / m->bs == id) slots_out[u] = -1;
          }
          row[j] = -1;
        }
        m->first[s] = j + 1;
      }
      int64_t lb = p / m->bs;
      if (lb >= m->max_blocks) return mgr_end_step(m, evicted_out, ne, ORC_INVALID_INPUT);
      if (p % m->bs == 0) {
        int64_t id = orc_pool_allocate(m->pool);
        if (id < 0) return mgr_end_step(m, evicted_out, ne, ORC_INVALID_INPUT); /* pool exhausted */
        row[lb] = (int32_t)id;
      } else if (row[lb] < 0) {
        return mgr_end_step(m, evicted_out, ne, ORC_INVALID_INPUT);
      } else if (cow && orc_pool_ref_count(m->pool, row[lb]) > 1) {
        /* Copy-on-write: the token would write into a partial block another
         * sequence also holds.  A fresh block takes the copy; this sequence
         * drops its reference to the shared one. */
        if (nc >= cow_cap) return mgr_end_step(m, evicted_out, ne, ORC_INVALID_INPUT);
        int64_t id = orc_pool_allocate(m->pool);
        if (id < 0) return mgr_end_step(m, evicted_out, ne, ORC_INVALID_INPUT);
        cow_src[nc] = row[lb];
        cow_dst[nc] = (int32_t)id;
        ++nc;
        if (mgr_drop_ref(m->pool, row[lb]) < 1) return mgr_end_step(m, evicted_out, ne, ORC_INVALID_INPUT);
        row[lb] = (int32_t)id;
      }
      slots_out[t++] = (int64_t)row[lb] * m->bs + p % m->bs;
      m->pos[s] = p + 1;
    }
  }
  *n_evicted = ne;
  if (n_cow) *n_cow = nc;
  return mgr_end_step(m, evicted_out, ne, ORC_OK);
}

int orc_mgr_append(orc_kv_manager* m, const int32_t* seqs, const int32_t* n_tokens, int32_t n,
                   int64_t* slots_out, int32_t* evicted_out, int32_t evicted_cap,
                   int32_t* n_evicted) {
  return orc_mgr_append_cow(m, seqs, n_tokens, n, 0, slots_out, evicted_out, evicted_cap, n_evicted, NULL,
                            NULL, 0, NULL);
}

int orc_mgr_fork(orc_kv_manager* m, int32_t src, int32_t dst) {
  /* dst takes src's blocks (BlockPool::share, paged.rs:44-46 each) and its
   * position; dst must hold nothing. */
  if (src < 0 || src >= m->max_seqs || dst < 0 || dst >= m->max_seqs || src == dst) return ORC_INVALID_INPUT;
  int32_t* drow = m->table + (size_t)dst * m->max_blocks;
  const int32_t* srow = m->table + (size_t)src * m->max_blocks;
  for (int32_t j = 0; j < m->max_blocks; ++j)
    if (drow[j] >= 0) return ORC_INVALID_INPUT;
  for (int32_t j = 0; j < m->max_blocks; ++j) {
    if (srow[j] < 0) continue;
    if (orc_pool_share(m->pool, srow[j])) return ORC_INVALID_INPUT;
    drow[j] = srow[j];
  }
  m->pos[dst] = m->pos[src];
  m->first[dst] = m->first[src];
  return ORC_OK;
}

int orc_mgr_release(orc_kv_manager* m, int32_t s, int32_t* evicted_out, int32_t evicted_cap,
                    int32_t* n_evicted) {
  /* Every held block, lowest logical block first, drops this sequence's
   * reference; the blocks whose refcount reaches 0 are reported. */
  if (s < 0 || s >= m->max_seqs) return ORC_INVALID_INPUT;
  int32_t* row = m->table + (size_t)s * m->max_blocks;
  int32_t ne = 0;
  for (int32_t j = 0; j < m->max_blocks; ++j) {
    if (row[j] < 0) continue;
    int32_t id = row[j];
    if (orc_pool_free(m->pool, id)) return ORC_INVALID_INPUT;
    if (orc_pool_ref_count(m->pool, id) == 0) {
      if (ne >= evicted_cap) return ORC_INVALID_INPUT;
      evicted_out[ne++] = id;
    }
    row[j] = -1;
  }
  m->pos[s] = 0;
  m->first[s] = 0;
  *n_evicted = ne;
  return ORC_OK;
}

int orc_mgr_tables(const orc_kv_manager* m, int32_t* tables, int32_t max_blocks,
                   int32_t* ctx_lens, int32_t* start_pos) {
  if (max_blocks < m->max_blocks) return ORC_INVALID_INPUT;
  for (int32_t s = 0; s < m->max_seqs; ++s) {
    for (int32_t j = 0; j < max_blocks; ++j)
      tables[(size_t)s * max_blocks + j] = j < m->max_blocks ? m->table[(size_t)s * m->max_blocks + j] : -1;
    if (ctx_lens) ctx_lens[s] = (int32_t)m->pos[s];
    if (start_pos) {
      int64_t st = m->window > 0 ? m->pos[s] - m->window : 0;
      start_pos[s] = (int32_t)(st > 0 ? st : 0);
    }
  }
  return ORC_OK;
}
