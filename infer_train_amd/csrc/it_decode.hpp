// it_decode.hpp -- paged split-K flash-decode for gfx950 (device code).
//
// One workgroup (4 wave64s) owns one (sequence, KV head, head chunk,
// partition of P tokens).  The GC query heads of the chunk share every K/V
// byte the workgroup reads, so each KV page is read from HBM once per
// partition.  Three phases, separated by workgroup barriers:
//
//  1. QK.  A token row is split over L_QK lanes; each lane loads its slice
//     of the key with 16-byte (8-byte for Q8_0) vector loads straight from
//     the page the block table names (a wave instruction covers whole
//     128-byte lines), forms GC partial dot products (v_dot2_f32_bf16 /
//     _f16 on packed 16-bit data, fp32 FMA otherwise) and sums them across
//     the L_QK lanes with DPP row operations.  Scaled scores (log2 domain)
//     go to LDS.
//  2. Softmax statistics.  Per head, the partition max and sum of
//     exp2(s - max) are wavefront reductions (DPP within rows, ds_swizzle
//     and a bpermute across rows); the probabilities replace the scores in
//     LDS.  The max is exact for the partition, so no rescaling is needed
//     inside it.
//  3. PV.  A value row is split over L_PV lanes; each lane accumulates
//     GC x DPV fp32 outputs over its tokens; the partial sums are reduced
//     across lanes (swizzle/bpermute) and across the four waves (LDS).
//
// The partition's (m, l, O) go to the workspace; a second kernel merges the
// partitions: M = max m_p, L = sum l_p 2^(m_p-M), O = sum O_p 2^(m_p-M) / L,
// the split-K form of flash_attn_f32's online rescaling
// (src/backend/arm/flash_attn.rs:42-63, final 1/s at :66-71).
#pragma once
#include <hip/hip_runtime.h>

#include "it_device.hpp"
#include "it_kv.h"

namespace itkv {

struct DecodeArgs {
  const void* q;            // [n_seqs][n_heads][D]
  const char* k_pool;
  const char* v_pool;
  const int32_t* bt;        // [n_seqs][max_blocks], NULL = identity
  const int32_t* ctx_lens;  // NULL = ctx_const for every sequence
  const int32_t* start_pos; // NULL = 0
  const float* mask;        // additive mask by position, NULL = none
  float* ws_o;              // [n_seqs][n_heads][max_parts][D]
  float* ws_ml;             // [n_seqs][n_heads][max_parts][2]
  uint32_t* err;
  int64_t page_bytes;
  int64_t num_blocks;
  float scale_log2;         // softmax scale * log2(e)
  float scale;              // softmax scale (mask path)
  int ctx_const;
  int max_blocks;
  int n_heads;
  int n_kv_heads;
  int group;                // n_heads / n_kv_heads
  int chunks;               // head chunks per KV head (group / GC)
  int log2_bs;
  int partition;            // tokens per split, multiple of 64
  int max_parts;
};

template <int DT> struct KvTraits;
template <> struct KvTraits<IT_BF16> {
  static constexpr int kElemBytes = 2, kQkDims = 16, kPvDims = 8;
};
template <> struct KvTraits<IT_F16> {
  static constexpr int kElemBytes = 2, kQkDims = 16, kPvDims = 8;
};
template <> struct KvTraits<IT_F32> {
  static constexpr int kElemBytes = 4, kQkDims = 8, kPvDims = 4;
};
template <> struct KvTraits<IT_Q8_0> {
  static constexpr int kElemBytes = 1, kQkDims = 8, kPvDims = 8;
};

constexpr int kDecodeThreads = 256;
constexpr int kDecodeWaves = kDecodeThreads / 64;
constexpr int kMaxTablePerPart = 4096 / 8 + 2;  // partition <= 4096, block_size >= 8
constexpr float kLog2e = 1.4426950408889634f;

// Widen 8 packed 16-bit values (uint4) to float.
template <int DT>
__device__ __forceinline__ void widen8(const uint4& w, float* f) {
  const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (DT == IT_BF16) {
      f[2 * i] = bf16_lo(a[i]);
      f[2 * i + 1] = bf16_hi(a[i]);
    } else {
      f[2 * i] = f16_bits_to_f32(a[i] & 0xFFFFu);
      f[2 * i + 1] = f16_bits_to_f32(a[i] >> 16);
    }
  }
}

__device__ __forceinline__ float i8f(uint32_t w, int j) { return float(int32_t(w << (24 - 8 * j)) >> 24); }

template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == IT_BF16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a), __builtin_bit_cast(bf2, b), c, false);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
  }
}

template <int DT, int D, int GC>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_split(DecodeArgs a) {
  using T = KvTraits<DT>;
  constexpr int DPL = T::kQkDims;          // dims per lane, QK phase
  constexpr int LQ = D / DPL;              // lanes per token, QK phase
  constexpr int RQ = 64 / LQ;              // tokens per wave row, QK phase
  constexpr int DPV = T::kPvDims;          // dims per lane, PV phase
  constexpr int LV = D / DPV;              // lanes per token, PV phase
  constexpr int RV = 64 / LV;              // tokens per wave row, PV phase
  constexpr int ROW_BYTES = DT == IT_Q8_0 ? D : D * T::kElemBytes;
  static_assert(LQ >= 8 && LQ <= 64 && LV >= 16 && LV <= 64, "bad lane split");

  extern __shared__ float smem[];           // scores/probs [GC][P], then reduction
  __shared__ int32_t s_pages[kMaxTablePerPart];

  const int part = blockIdx.x;
  const int kvh = blockIdx.y / a.chunks;
  const int chunk = blockIdx.y - kvh * a.chunks;
  const int b = blockIdx.z;
  const int head0 = kvh * a.group + chunk * GC;

  const int ctx = a.ctx_lens ? a.ctx_lens[b] : a.ctx_const;
  const int st = a.start_pos ? a.start_pos[b] : 0;
  const int n = ctx - st;
  const int P = a.partition;
  if (n <= 0 || part * P >= n) return;  // uniform for the workgroup
  if (part == a.max_parts - 1 && n > a.max_parts * P && threadIdx.x == 0)
    atomicOr(a.err, 8u);  // context longer than the caller's max_tokens: tail ignored
  const int tok0 = st + part * P;
  const int nt = min(P, n - part * P);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bs_mask = (1 << a.log2_bs) - 1;

  // Page indices (block * n_kv_heads + kvh) of the partition, via LDS.
  const int lb0 = tok0 >> a.log2_bs;
  const int nlb = ((tok0 + nt - 1) >> a.log2_bs) - lb0 + 1;
  for (int i = tid; i < nlb; i += kDecodeThreads) {
    const int lb = lb0 + i;
    int blk = lb;
    if (a.bt) {
      if (lb >= a.max_blocks) {
        atomicOr(a.err, 4u);
        blk = 0;
      } else {
        blk = a.bt[int64_t(b) * a.max_blocks + lb];
      }
    }
    if (blk < 0 || blk >= a.num_blocks) {
      atomicOr(a.err, 2u);
      blk = 0;
    }
    s_pages[i] = blk * a.n_kv_heads + kvh;
  }
  __syncthreads();

  float* s_sc = smem;  // [GC][P]

  // ---------------- phase 1: scores --------------------------------------
  {
    const int li = lane % LQ, tj = lane / LQ;
    const int64_t qrow = (int64_t(b) * a.n_heads + head0) * D;
    if constexpr (DT == IT_BF16 || DT == IT_F16) {
      // Lane slice: dims [8li, 8li+8) and [D/2 + 8li, D/2 + 8li + 8).
      uint32_t qr[GC][8];
      const uint16_t* qp = static_cast<const uint16_t*>(a.q) + qrow;
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        const uint4 q0 = ld16(qp + g * D + 8 * li);
        const uint4 q1 = ld16(qp + g * D + D / 2 + 8 * li);
        qr[g][0] = q0.x; qr[g][1] = q0.y; qr[g][2] = q0.z; qr[g][3] = q0.w;
        qr[g][4] = q1.x; qr[g][5] = q1.y; qr[g][6] = q1.z; qr[g][7] = q1.w;
      }
      const int nrows = (nt + RQ - 1) / RQ;
      for (int r = wave; r < nrows; r += kDecodeWaves) {
        const int tr = r * RQ + tj;
        const bool valid = tr < nt;
        const int t = tok0 + (valid ? tr : 0);
        const char* row = a.k_pool + int64_t(s_pages[(t >> a.log2_bs) - lb0]) * a.page_bytes +
                          int64_t(t & bs_mask) * ROW_BYTES;
        const uint4 k0 = ld16(row + 16 * li);
        const uint4 k1 = ld16(row + D + 16 * li);
        const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
        float sc[GC];
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          float acc = 0.0f;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc = dot2<DT>(kw[j], qr[g][j], acc);
          sc[g] = group_sum<LQ>(acc);
        }
        if (li == 0 && valid) {
#pragma unroll
          for (int g = 0; g < GC; ++g) {
            float s = sc[g] * a.scale_log2;
            if (a.mask) {
              const float mk = a.mask[t];
              s = (mk == -INFINITY) ? -INFINITY : (sc[g] * a.scale + mk) * kLog2e;
            }
            s_sc[g * P + tr] = s;
          }
        }
      }
    } else {
      // F32 or Q8_0: fp32 q, slice [4li, 4li+4) and [D/2 + 4li, ...) for F32;
      // [8li, 8li+8) for Q8_0 (one 32-group per 4 lanes).
      float qf[GC][8];
      const float* qp = static_cast<const float*>(a.q) + qrow;
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        float4 q0, q1;
        if constexpr (DT == IT_F32) {
          q0 = *reinterpret_cast<const float4*>(qp + g * D + 4 * li);
          q1 = *reinterpret_cast<const float4*>(qp + g * D + D / 2 + 4 * li);
        } else {
          q0 = *reinterpret_cast<const float4*>(qp + g * D + 8 * li);
          q1 = *reinterpret_cast<const float4*>(qp + g * D + 8 * li + 4);
        }
        qf[g][0] = q0.x; qf[g][1] = q0.y; qf[g][2] = q0.z; qf[g][3] = q0.w;
        qf[g][4] = q1.x; qf[g][5] = q1.y; qf[g][6] = q1.z; qf[g][7] = q1.w;
      }
      const int nrows = (nt + RQ - 1) / RQ;
      for (int r = wave; r < nrows; r += kDecodeWaves) {
        const int tr = r * RQ + tj;
        const bool valid = tr < nt;
        const int t = tok0 + (valid ? tr : 0);
        const char* page = a.k_pool + int64_t(s_pages[(t >> a.log2_bs) - lb0]) * a.page_bytes;
        const int off = t & bs_mask;
        float kf[8];
        float dsc = 1.0f;
        if constexpr (DT == IT_F32) {
          const float4 k0 = *reinterpret_cast<const float4*>(page + int64_t(off) * ROW_BYTES + 16 * li);
          const float4 k1 = *reinterpret_cast<const float4*>(page + int64_t(off) * ROW_BYTES + 2 * D + 16 * li);
          kf[0] = k0.x; kf[1] = k0.y; kf[2] = k0.z; kf[3] = k0.w;
          kf[4] = k1.x; kf[5] = k1.y; kf[6] = k1.z; kf[7] = k1.w;
        } else {
          const uint2 w = *reinterpret_cast<const uint2*>(page + int64_t(off) * D + 8 * li);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            kf[j] = i8f(w.x, j);
            kf[4 + j] = i8f(w.y, j);
          }
          const int64_t bs = int64_t(bs_mask) + 1;
          dsc = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(page + bs * D + (int64_t(off) * (D / 32) + li / 4) * 2));
        }
        float sc[GC];
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          float acc = 0.0f;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc = fmaf(qf[g][j], kf[j], acc);
          if constexpr (DT == IT_Q8_0) acc *= dsc;  // x = f32(d) * q (gemv.rs:151-160)
          sc[g] = group_sum<LQ>(acc);
        }
        if (li == 0 && valid) {
#pragma unroll
          for (int g = 0; g < GC; ++g) {
            float s = sc[g] * a.scale_log2;
            if (a.mask) {
              const float mk = a.mask[t];
              s = (mk == -INFINITY) ? -INFINITY : (sc[g] * a.scale + mk) * kLog2e;
            }
            s_sc[g * P + tr] = s;
          }
        }
      }
    }
  }
  __syncthreads();

  // ---------------- phase 2: softmax statistics ---------------------------
  const int64_t part_row = (int64_t(b) * a.n_heads + head0) * a.max_parts + part;
  for (int g = wave; g < GC; g += kDecodeWaves) {
    float mx = -INFINITY;
    for (int i = lane; i < nt; i += 64) mx = fmaxf(mx, s_sc[g * P + i]);
    mx = group_max<64>(mx);
    float sum = 0.0f;
    for (int i = lane; i < nt; i += 64) {
      const float p = (mx == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s_sc[g * P + i] - mx);
      s_sc[g * P + i] = p;
      sum += p;
    }
    sum = group_sum<64>(sum);
    if (lane == 0) {
      float* ml = a.ws_ml + (part_row + int64_t(g) * a.max_parts) * 2;
      ml[0] = mx;
      ml[1] = sum;
    }
  }
  __syncthreads();

  // ---------------- phase 3: P.V ----------------------------------------
  float acc[GC][DPV];
#pragma unroll
  for (int g = 0; g < GC; ++g)
#pragma unroll
    for (int j = 0; j < DPV; ++j) acc[g][j] = 0.0f;
  {
    const int li = lane % LV, tj = lane / LV;
    const int nrows = (nt + RV - 1) / RV;
    for (int r = wave; r < nrows; r += kDecodeWaves) {
      const int tr = r * RV + tj;
      const bool valid = tr < nt;
      const int t = tok0 + (valid ? tr : 0);
      const char* page = a.v_pool + int64_t(s_pages[(t >> a.log2_bs) - lb0]) * a.page_bytes;
      const int off = t & bs_mask;
      float vf[DPV];
      float dsc = 1.0f;
      if constexpr (DT == IT_BF16 || DT == IT_F16) {
        widen8<DT>(ld16(page + int64_t(off) * ROW_BYTES + 16 * li), vf);
      } else if constexpr (DT == IT_F32) {
        const float4 v4 = *reinterpret_cast<const float4*>(page + int64_t(off) * ROW_BYTES + 16 * li);
        vf[0] = v4.x; vf[1] = v4.y; vf[2] = v4.z; vf[3] = v4.w;
      } else {
        const uint2 w = *reinterpret_cast<const uint2*>(page + int64_t(off) * D + 8 * li);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          vf[j] = i8f(w.x, j);
          vf[4 + j] = i8f(w.y, j);
        }
        const int64_t bs = int64_t(bs_mask) + 1;
        dsc = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(page + bs * D + (int64_t(off) * (D / 32) + li / 4) * 2));
      }
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        float p = valid ? s_sc[g * P + tr] : 0.0f;
        if constexpr (DT == IT_Q8_0) p *= dsc;  // p * (d * q) = (p * d) * q
#pragma unroll
        for (int j = 0; j < DPV; ++j) acc[g][j] = fmaf(p, vf[j], acc[g][j]);
      }
    }
  }
  // Reduce over the RV token slots of the wave (lanes li, li+LV, ...).
#pragma unroll
  for (int g = 0; g < GC; ++g)
#pragma unroll
    for (int j = 0; j < DPV; ++j) {
      float x = acc[g][j];
      if constexpr (LV <= 16) x += swz_xor16(x);
      if constexpr (LV <= 32) x += swap_halves(x);
      acc[g][j] = x;
    }
  __syncthreads();  // everyone is done with the probabilities
  float* s_red = smem;  // [waves][GC][D]
  {
    const int li = lane % LV, tj = lane / LV;
    if (tj == 0) {
#pragma unroll
      for (int g = 0; g < GC; ++g)
#pragma unroll
        for (int j = 0; j < DPV; ++j) {
          // PV slice of lane li: dims [DPV*li, DPV*li + DPV)
          s_red[(wave * GC + g) * D + DPV * li + j] = acc[g][j];
        }
    }
  }
  __syncthreads();
  for (int i = tid; i < GC * D; i += kDecodeThreads) {
    float o = s_red[i];
#pragma unroll
    for (int w = 1; w < kDecodeWaves; ++w) o += s_red[w * GC * D + i];
    const int g = i / D, d = i - g * D;
    a.ws_o[(part_row + int64_t(g) * a.max_parts) * D + d] = o;
  }
}

// Merge the partitions of one (sequence, head).  64 lanes; lane owns D/64
// output dims.
template <int D>
__global__ __launch_bounds__(64) void paged_decode_combine(const float* __restrict__ ws_o,
                                                           const float* __restrict__ ws_ml,
                                                           const int32_t* __restrict__ ctx_lens,
                                                           const int32_t* __restrict__ start_pos,
                                                           int ctx_const, int n_heads, int partition,
                                                           int max_parts, void* out, int out_dtype) {
  // Partitions beyond max_parts were never computed (the split pass latched
  // the error); only the computed ones are merged.
  constexpr int DL = D / 64;
  __shared__ float s_w[4096];
  const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int ctx = ctx_lens ? ctx_lens[b] : ctx_const;
  const int st = start_pos ? start_pos[b] : 0;
  const int n = ctx - st;
  const int np = n > 0 ? min((n + partition - 1) / partition, max_parts) : 0;
  const int64_t row = int64_t(b) * n_heads + h;
  const float* ml = ws_ml + row * max_parts * 2;
  float mx = -INFINITY;
  for (int p = lane; p < np; p += 64) mx = fmaxf(mx, ml[2 * p]);
  mx = group_max<64>(mx);
  float l = 0.0f;
  for (int p = lane; p < np; p += 64) {
    const float w = (mx == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ml[2 * p] - mx);
    s_w[p] = w;
    l += ml[2 * p + 1] * w;
  }
  l = group_sum<64>(l);
  __syncthreads();
  float o[DL];
#pragma unroll
  for (int j = 0; j < DL; ++j) o[j] = 0.0f;
  const float* op = ws_o + row * max_parts * D;
  for (int p = 0; p < np; ++p) {
    const float w = s_w[p];
#pragma unroll
    for (int j = 0; j < DL; ++j) o[j] = fmaf(op[int64_t(p) * D + lane + 64 * j], w, o[j]);
  }
  // flash_attn.rs:66-71: multiply by 1/s when s > 0, else zeros.
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
  for (int j = 0; j < DL; ++j) {
    const float v = l > 0.0f ? o[j] * inv : 0.0f;
    const int64_t idx = row * D + lane + 64 * j;
    if (out_dtype == IT_F32) static_cast<float*>(out)[idx] = v;
    else if (out_dtype == IT_BF16) static_cast<uint16_t*>(out)[idx] = uint16_t(f32_to_bf16_bits(v));
    else static_cast<uint16_t*>(out)[idx] = uint16_t(f32_to_f16_bits(v));
  }
}

}  // namespace itkv
