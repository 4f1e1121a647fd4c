// it_rope.hip -- RoPE then append (src/inference/forward.rs:195-229): the
// rotary embedding of q and k (rope_f32, src/backend/arm/rope.rs:6-44) fused
// into the slot-mapped KV append, so the rotated K goes straight from the
// projection output into its cache page in the cache's format.
//
// The angles' cos/sin come from a table built on the host with the C
// library's float32 powf/cosf/sinf, in rope_f32's operation order, and held
// on the device: the device only multiplies and adds, so its results equal
// the CPU's bit for bit.  One lane rotates one 16-byte vector (two pairs) of
// one (token, head) row; K and V lanes then convert (or quantise: Q8_0,
// Q4_0, Q4_1, Q5_0, Q5_1) and store like the plain append, Q lanes write the
// rotated query.
#include <hip/hip_runtime.h>

#include <cmath>
#include <vector>

#include "it_device.hpp"
#include "it_internal.hpp"
#include "it_quant.hpp"

using namespace itkv;

struct it_rope_table {
  float2* table;  // device [max_pos][n_dims / 2]: (cos, sin)
  int32_t device;
  int32_t n_dims;
  int32_t max_pos;
  float freq_base;
};

namespace {
constexpr int kThreads = 256;

struct RopeAppendArgs {
  const float4* q;
  const float4* k;
  const float4* v;
  void* q_out;
  char* kpool;
  char* vpool;
  const int64_t* slots;
  const int32_t* positions;
  const float2* table;
  int64_t n_tokens;
  int64_t page_bytes;
  int64_t n_slots;
  uint32_t* err;
  int hq, hkv, d, n_dims, max_pos, log2_bs, q_out_dtype;
};


// Four floats to the 16-bit format DT16 (IT_BF16 or IT_F16), packed.
template <int DT16>
__device__ __forceinline__ uint2 pack4(const float4& x) {
  auto cv = [](float f) { return DT16 == IT_BF16 ? f32_to_bf16_bits(f) : f16_bits_rne(f); };
  return make_uint2(cv(x.x) | (cv(x.y) << 16), cv(x.z) | (cv(x.w) << 16));
}


// rope.rs:38-39 on the pairs (x, y) and (z, w) with the table's (cos, sin):
// two products, each rounded, then their difference / sum -- no FMA.
__device__ __forceinline__ float4 rotate(float4 x, float2 cs0, float2 cs1, bool r0, bool r1) {
  float4 o = x;
  if (r0) {
    o.x = mul_rn(x.x, cs0.x) - mul_rn(x.y, cs0.y);
    o.y = mul_rn(x.x, cs0.y) + mul_rn(x.y, cs0.x);
  }
  if (r1) {
    o.z = mul_rn(x.z, cs1.x) - mul_rn(x.w, cs1.y);
    o.w = mul_rn(x.z, cs1.y) + mul_rn(x.w, cs1.x);
  }
  return o;
}

// grid.y: 0 = K, 1 = V, 2 = Q.  DT: the cache dtype.
template <int DT>
__global__ __launch_bounds__(kThreads) void kv_append_rope(RopeAppendArgs a) {
  const int part = blockIdx.y;
  const int H = part == 2 ? a.hq : a.hkv;
  const int vecs = a.d >> 2;
  const int64_t gid = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t total = a.n_tokens * H * vecs;
  const bool live = gid < total;
  const int cv = int(gid % vecs);
  const int64_t th = gid / vecs;
  const int h = int(th % H);
  const int64_t t = th / H;
  const float4* src = part == 0 ? a.k : (part == 1 ? a.v : a.q);
  float4 x = live ? src[gid] : make_float4(0.f, 0.f, 0.f, 0.f);
  // A token whose position is outside the table writes nothing (K, V or q).
  bool pos_ok = true;
  if (live) {
    const int pos = a.positions[t];
    pos_ok = pos >= 0 && pos < a.max_pos;
    if (!pos_ok) {
      if (cv == 0 && h == 0 && part == 0) atomicOr(a.err, kErrPos);
    } else if (part != 1) {
      // Elements 4 cv .. 4 cv + 3 are pairs 2 cv and 2 cv + 1.
      const int e0 = 4 * cv;
      const float2* row = a.table + int64_t(pos) * (a.n_dims >> 1) + 2 * cv;
      const bool r0 = e0 < a.n_dims, r1 = e0 + 2 < a.n_dims;
      const float2 cs0 = r0 ? row[0] : make_float2(1.f, 0.f);
      const float2 cs1 = r1 ? row[1] : make_float2(1.f, 0.f);
      x = rotate(x, cs0, cs1, r0, r1);
    }
  }
  if (part == 2) {
    if (!live || !pos_ok) return;
    if (a.q_out_dtype == IT_F32) static_cast<float4*>(a.q_out)[gid] = x;
    else if (a.q_out_dtype == IT_BF16) static_cast<uint2*>(a.q_out)[gid] = pack4<IT_BF16>(x);
    else static_cast<uint2*>(a.q_out)[gid] = pack4<IT_F16>(x);
    return;
  }
  if constexpr (DT == IT_Q8_0 || DT == IT_Q4_0 || DT == IT_Q4_1 || DT == IT_Q5_0 || DT == IT_Q5_1) {
    // Eight lanes own one 32-element group (rows of d/4 vectors, d % 32 ==
    // 0): the group's reductions run before any lane leaves.
    const QuantGroup qg = quant_group<DT>(x, cv & 7);
    if (!live || !pos_ok) return;
    const int64_t slot = a.slots[t];
    if (slot < 0) return;
    if (slot >= a.n_slots) {
      if (cv == 0 && h == 0) atomicOr(a.err, kErrSlot);
      return;
    }
    const int64_t blk = slot >> a.log2_bs;
    const int64_t off = slot & ((int64_t(1) << a.log2_bs) - 1);
    char* page = (part == 1 ? a.vpool : a.kpool) + (blk * a.hkv + h) * a.page_bytes;
    store_group<DT>(page, off, int64_t(1) << a.log2_bs, a.d, cv, qg);
  } else {
    if (!live || !pos_ok) return;
    const int64_t slot = a.slots[t];
    if (slot < 0) return;
    if (slot >= a.n_slots) {
      if (cv == 0 && h == 0) atomicOr(a.err, kErrSlot);
      return;
    }
    const int64_t blk = slot >> a.log2_bs;
    const int64_t off = slot & ((int64_t(1) << a.log2_bs) - 1);
    char* row = (part == 1 ? a.vpool : a.kpool) + (blk * a.hkv + h) * a.page_bytes;
    if constexpr (DT == IT_F32) {
      reinterpret_cast<float4*>(row + off * a.d * 4)[cv] = x;
    } else {
      reinterpret_cast<uint2*>(row + off * a.d * 2)[cv] = pack4<DT>(x);
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

extern "C" int32_t it_rope_table_new(int32_t device, int32_t n_dims, float freq_base, int32_t max_pos,
                                     it_rope_table** out) {
  const char* who = "it_rope_table_new";
  if (!out) return fail(IT_INVALID_INPUT, "%s: out is NULL", who);
  *out = nullptr;
  if (n_dims <= 0 || n_dims % 4 || n_dims > 4096)
    return fail(IT_INVALID_INPUT, "%s: n_dims %d must be a positive multiple of 4 (<= 4096)", who, n_dims);
  if (max_pos <= 0) return fail(IT_INVALID_INPUT, "%s: max_pos %d", who, max_pos);
  if (!(freq_base > 0.0f) || !std::isfinite(freq_base))
    return fail(IT_INVALID_INPUT, "%s: freq_base must be positive and finite", who);
  const int pairs = n_dims / 2;
  // rope.rs:30-34, float32: theta = (float)pos * powf(base, -(float)i / (float)n_dims).
  std::vector<float> inv(pairs);
  for (int p = 0; p < pairs; ++p) inv[p] = powf(freq_base, -float(2 * p) / float(n_dims));
  std::vector<float2> host(size_t(max_pos) * pairs);
  for (int64_t pos = 0; pos < max_pos; ++pos)
    for (int p = 0; p < pairs; ++p) {
      const float theta = float(pos) * inv[p];
      host[size_t(pos) * pairs + p] = make_float2(cosf(theta), sinf(theta));
    }
  int prev = -1;
  (void)hipGetDevice(&prev);
  if (hipSetDevice(device) != hipSuccess) return fail(IT_DEVICE_ERROR, "%s: hipSetDevice(%d)", who, device);
  float2* dev = nullptr;
  hipError_t e = hipMalloc(&dev, host.size() * sizeof(float2));
  if (e == hipSuccess) e = hipMemcpy(dev, host.data(), host.size() * sizeof(float2), hipMemcpyHostToDevice);
  if (prev >= 0) (void)hipSetDevice(prev);
  if (e != hipSuccess) {
    if (dev) (void)hipFree(dev);
    return fail(IT_DEVICE_ERROR, "%s: %s", who, hipGetErrorString(e));
  }
  *out = new it_rope_table{dev, device, n_dims, max_pos, freq_base};
  return IT_OK;
}

extern "C" int32_t it_rope_table_destroy(it_rope_table* r) {
  if (!r) return IT_OK;
  int prev = -1;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(r->device);
  const hipError_t e = hipFree(r->table);
  if (prev >= 0) (void)hipSetDevice(prev);
  delete r;
  return e == hipSuccess ? IT_OK : fail(IT_DEVICE_ERROR, "it_rope_table_destroy: %s", hipGetErrorString(e));
}

extern "C" int32_t it_kv_append_rope(it_kv_cache* c, const it_rope_table* rope, const float* q, int32_t n_heads,
                                     const float* k, const float* v, const int64_t* slot_mapping,
                                     const int32_t* positions, int32_t n_tokens, void* q_out, int32_t q_out_dtype,
                                     void* stream) {
  const char* who = "it_kv_append_rope";
  if (!c || !rope) return fail(IT_INVALID_INPUT, "%s: cache or table is NULL", who);
  if (int32_t rc = one_layer(c, who)) return rc;
  if (n_tokens < 0) return fail(IT_INVALID_INPUT, "%s: n_tokens %d < 0", who, n_tokens);
  if (n_heads <= 0 || n_heads % c->n_kv_heads)
    return fail(IT_INVALID_INPUT, "%s: n_heads %d must be a positive multiple of n_kv_heads %d", who, n_heads,
                c->n_kv_heads);
  if (rope->n_dims > c->head_dim)
    return fail(IT_INVALID_INPUT, "%s: table n_dims %d > head_dim %d", who, rope->n_dims, c->head_dim);
  if (rope->device != c->device) return fail(IT_INVALID_INPUT, "%s: table and cache on different devices", who);
  const bool quant = is_quant(c->dtype);
  if (c->dtype != IT_F32 && c->dtype != IT_BF16 && c->dtype != IT_F16 && !quant)
    return fail(IT_NOT_IMPLEMENTED, "%s: cache dtype %d", who, c->dtype);
  const bool q_ok = q_out_dtype == IT_F32 || ((c->dtype == IT_BF16 || c->dtype == IT_F16) && q_out_dtype == c->dtype);
  if (!q_ok) return fail(IT_NOT_IMPLEMENTED, "%s: q_out dtype %d for cache dtype %d", who, q_out_dtype, c->dtype);
  if (c->head_dim % 4 || (quant && c->head_dim % 32))
    return fail(IT_NOT_IMPLEMENTED, "%s: head_dim %d", who, c->head_dim);
  if (n_tokens == 0) return IT_OK;
  if (!q || !k || !v || !slot_mapping || !positions || !q_out) return fail(IT_INVALID_INPUT, "%s: NULL tensor", who);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(q_out))
    return fail(IT_INVALID_INPUT, "%s: q/k/v/q_out must be 16-byte aligned", who);
  RopeAppendArgs a{};
  a.q = reinterpret_cast<const float4*>(q);
  a.k = reinterpret_cast<const float4*>(k);
  a.v = reinterpret_cast<const float4*>(v);
  a.q_out = q_out;
  a.kpool = static_cast<char*>(c->k_pool);
  a.vpool = static_cast<char*>(c->v_pool);
  a.slots = slot_mapping;
  a.positions = positions;
  a.table = rope->table;
  a.n_tokens = n_tokens;
  a.page_bytes = c->page_bytes;
  a.n_slots = c->num_blocks * c->block_size;
  a.err = c->err_flag;
  a.hq = n_heads;
  a.hkv = c->n_kv_heads;
  a.d = c->head_dim;
  a.n_dims = rope->n_dims;
  a.max_pos = rope->max_pos;
  a.log2_bs = c->log2_bs;
  a.q_out_dtype = q_out_dtype;
  const int64_t vecs = int64_t(n_tokens) * n_heads * (c->head_dim / 4);  // Q has the most rows
  const int64_t blocks = (vecs + kThreads - 1) / kThreads;
  if (blocks > INT32_MAX) return fail(IT_INVALID_INPUT, "%s: too many tokens", who);
  int dev = -1;
  (void)hipGetDevice(&dev);
  if (dev != c->device) (void)hipSetDevice(c->device);
  const dim3 grid(unsigned(blocks), 3);
  hipStream_t s = (hipStream_t)stream;
  switch (c->dtype) {
    case IT_F32: hipLaunchKernelGGL(kv_append_rope<IT_F32>, grid, dim3(kThreads), 0, s, a); break;
    case IT_BF16: hipLaunchKernelGGL(kv_append_rope<IT_BF16>, grid, dim3(kThreads), 0, s, a); break;
    case IT_F16: hipLaunchKernelGGL(kv_append_rope<IT_F16>, grid, dim3(kThreads), 0, s, a); break;
    case IT_Q4_0: hipLaunchKernelGGL(kv_append_rope<IT_Q4_0>, grid, dim3(kThreads), 0, s, a); break;
    case IT_Q4_1: hipLaunchKernelGGL(kv_append_rope<IT_Q4_1>, grid, dim3(kThreads), 0, s, a); break;
    case IT_Q5_0: hipLaunchKernelGGL(kv_append_rope<IT_Q5_0>, grid, dim3(kThreads), 0, s, a); break;
    case IT_Q5_1: hipLaunchKernelGGL(kv_append_rope<IT_Q5_1>, grid, dim3(kThreads), 0, s, a); break;
    default: hipLaunchKernelGGL(kv_append_rope<IT_Q8_0>, grid, dim3(kThreads), 0, s, a); break;
  }
  const hipError_t e = hipGetLastError();
  if (dev >= 0 && dev != c->device) (void)hipSetDevice(dev);
  if (e != hipSuccess) return fail(IT_DEVICE_ERROR, "%s: launch: %s", who, hipGetErrorString(e));
  return IT_OK;
}
