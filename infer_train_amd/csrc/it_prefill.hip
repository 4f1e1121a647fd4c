// it_prefill.hip -- chunked-prefill attention over the paged cache, on MFMA.
//
// A chunk of q_len query rows per sequence, at positions ctx - q_len + i,
// attends (causally, or over the whole context) the keys in the paged cache
// (the chunk's own K/V already appended).  Per query row this is
// flash_attn_f32 (src/backend/arm/flash_attn.rs:6-72) over keys
// 0..ctx - q_len + i, with the GQA map of src/inference/forward.rs:231-254;
// the chunked prefill itself has no counterpart in the reference, whose
// generate loop feeds one token at a time (forward.rs:811).
//
// One workgroup = (sequence, KV head, block of 32 query positions); wave w
// handles query head kvh * G + w for those 32 positions, so the G waves of a
// group share every K/V byte the workgroup reads.  Per 64-key block:
//   S^T = K Q^T   v_mfma_f32_32x32x16 (keys are MFMA rows, queries columns),
//                 so each lane owns one query column: its row max and sum
//                 are in-lane (plus one exchange with lane ^ 32);
//   O^T += V^T P^T the probabilities go back into MFMA operands straight
//                 from the S^T registers (bf16/f16), and V^T comes from the
//                 row-major V tile through ds_read_b64_tr_b16 transposing
//                 loads; the contraction runs over keys in the order the S^T
//                 registers hold them, and the V^T loads follow that order.
// K and V blocks (16 KiB each) are staged in LDS by direct global->LDS loads,
// 16-byte chunks XOR-swizzled by row so MFMA operand reads are conflict-free,
// double-buffered: block j+1 loads while block j is computed.  Online
// softmax in fp32 (exp2 domain), accumulators fp32.
#include <hip/hip_runtime.h>

#include "it_device.hpp"
#include "it_internal.hpp"

using namespace itkv;

namespace {
constexpr int kD = 128;           // head_dim
constexpr int kQB = 32;           // query positions per workgroup
constexpr int kKB = 64;           // keys per block
constexpr int kRowB = kD * 2;     // bytes per K/V row
constexpr int kPlaneB = kKB * kRowB;  // 16 KiB
constexpr int kStageB = 2 * kPlaneB;  // K + V
constexpr int kMaxGroup = 8;      // waves per workgroup (512 threads)

typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct PrefillArgs {
  const uint16_t* q;      // [total_q][n_heads][D]
  const char* k_pool;
  const char* v_pool;
  const int32_t* cu_q;    // [n_seqs + 1]
  const int32_t* bt;      // [n_seqs][max_blocks]
  const int32_t* ctx_lens;
  void* out;              // [total_q][n_heads][D]
  uint32_t* err;
  int64_t page_bytes;
  int64_t num_blocks;
  float scale_log2;
  int n_heads, n_kv_heads, group, max_blocks, log2_bs, causal, out_f32;
};

__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}
__device__ __forceinline__ void dma_b128(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(g) : "memory", "m0");
}
// Byte offset of 16-byte chunk c of row r in a swizzled tile.
__device__ __forceinline__ int swz(int r, int c) { return r * kRowB + ((c ^ (r & 7)) << 4); }

template <bool kBf16>
__device__ __forceinline__ v16f mfma(const uint4& a, const uint4& b, const v16f& c) {
  if constexpr (kBf16) {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  } else {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
}
template <bool kBf16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (kBf16) return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
  else return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
}

// MAXW: the largest group this instantiation serves (sets the register budget).
template <bool kBf16, int MAXW>
__global__ __launch_bounds__(64 * MAXW) __attribute__((amdgpu_waves_per_eu(2)))
void paged_prefill_kernel(PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];  // 2 stages x (K tile, V tile)
  const int qb = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int q_begin = a.cu_q[b];
  const int q_len = a.cu_q[b + 1] - q_begin;
  const int ctx = a.ctx_lens[b];
  if (qb * kQB >= q_len) return;  // uniform
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = a.group;
  const int head = kvh * a.group + wave;
  const int half = lane >> 5;  // 0 / 1
  const int col = lane & 31;   // this lane's query within the block
  const int qi = qb * kQB + col;
  const bool q_ok = qi < q_len;
  const int q_pos = ctx - q_len + qi;  // absolute position of this lane's query
  // Keys this workgroup needs: up to the last valid query's position.
  const int last_q = min(q_len, (qb + 1) * kQB) - 1;
  const int kend = a.causal ? min(ctx, ctx - q_len + last_q + 1) : ctx;
  const int nkb = (kend + kKB - 1) / kKB;

  // q: B operand of S^T = K Q^T, k-step ks holds dims 16 ks + 8 half + [0, 8).
  uint4 qv[kD / 16];
  {
    const uint16_t* qp = a.q + ((int64_t(q_begin) + (q_ok ? qi : 0)) * a.n_heads + head) * kD + 8 * half;
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks) {
      qv[ks] = q_ok ? ld16(qp + 16 * ks) : make_uint4(0u, 0u, 0u, 0u);
      asm volatile("" : "+v"(qv[ks].x), "+v"(qv[ks].y), "+v"(qv[ks].z), "+v"(qv[ks].w));
    }
  }

  const int bs_mask = (1 << a.log2_bs) - 1;
  const int32_t* bt = a.bt + int64_t(b) * a.max_blocks;
  // Loads of key block kb into stage st: 32 1-KiB instructions (K then V),
  // spread over the waves.  Lane l of instruction i covers tile row
  // 4 (i % 16) + l / 16 and, swizzled, global chunk (l % 16) ^ (row & 7).
  auto issue = [&](int kb, int st) {
    for (int i = wave; i < 32; i += nw) {
      const int plane = i >> 4;
      const int row = 4 * (i & 15) + (lane >> 4);
      const int chunk = (lane & 15) ^ (row & 7);
      int key = kb * kKB + row;
      if (key >= kend) key = kend - 1;  // rows past the keys: a valid row, masked out later
      const int lb = key >> a.log2_bs;
      int blk = lb < a.max_blocks ? bt[lb] : -1;
      if (blk < 0 || blk >= a.num_blocks) {
        atomicOr(a.err, 2u);
        blk = 0;
      }
      const char* pool = plane ? a.v_pool : a.k_pool;
      const char* g = pool + (int64_t(blk) * a.n_kv_heads + kvh) * a.page_bytes + int64_t(key & bs_mask) * kRowB + chunk * 16;
      dma_b128(g, __builtin_amdgcn_readfirstlane(lds_off(smem) + uint32_t(st * kStageB + plane * kPlaneB + (i & 15) * 1024)));
    }
  };

  v16f o[kD / 32];
#pragma unroll
  for (int d = 0; d < kD / 32; ++d) o[d] = v16f{};
  float m_run = -INFINITY, l_run = 0.0f;

  if (nkb > 0) issue(0, 0);
  for (int kb = 0; kb < nkb; ++kb) {
    const int st = kb & 1;
    // Block kb has landed (this wave's loads; the barrier makes it everyone's,
    // and frees stage st^1, read at kb-1, for block kb+1).
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (kb + 1 < nkb) issue(kb + 1, st ^ 1);
    const char* kt = smem + st * kStageB;
    const char* vt = kt + kPlaneB;

    // ---- S^T for two 32-key tiles -------------------------------------------
    v16f s[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      s[n] = v16f{};
#pragma unroll
      for (int ks = 0; ks < kD / 16; ++ks) {
        // A: key row 32 n + col, dims 16 ks + 8 half + [0, 8) = chunk 2 ks + half.
        const uint4 kk = *reinterpret_cast<const uint4*>(kt + swz(32 * n + col, 2 * ks + half));
        s[n] = mfma<kBf16>(kk, qv[ks], s[n]);
      }
    }
    // ---- online softmax (fp32, log2 domain) ----------------------------------
    // s[n][r] is key 64 kb + 32 n + 8 (r / 4) + 4 half + r % 4 for query col.
    float bmax = -INFINITY;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb * kKB + 32 * n + 8 * (r >> 2) + 4 * half + (r & 3);
        const bool ok = key < kend && (!a.causal || key <= q_pos);
        const float x = ok ? s[n][r] * a.scale_log2 : -INFINITY;
        s[n][r] = x;
        bmax = fmaxf(bmax, x);
      }
    bmax = fmaxf(bmax, swap_halves(bmax));
    const float m_new = fmaxf(m_run, bmax);
    const bool none = m_new == -INFINITY;
    const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    float bsum = 0.0f;
    uint4 pk[2][2];  // [tile][k-step]: 8 probabilities each, packed
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          p[e] = none ? 0.0f : __builtin_amdgcn_exp2f(s[n][8 * t + e] - m_new);
          bsum += p[e];
        }
        pk[n][t] = make_uint4(pack2<kBf16>(p[0], p[1]), pack2<kBf16>(p[2], p[3]), pack2<kBf16>(p[4], p[5]),
                              pack2<kBf16>(p[6], p[7]));
      }
    l_run = l_run * alpha + bsum;
    m_run = m_new;
#pragma unroll
    for (int d = 0; d < kD / 32; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[d][r] *= alpha;

    // ---- O^T += V^T P^T ------------------------------------------------------
    // k-step (n, t), element e of lane half h <-> key 32 n + 16 t + 8 (e / 4)
    // + 4 h + e % 4: the keys s[n][8 t + e] holds.  Transposing load c
    // (e = 4 c + j) of lane L reads key 32 n + 16 t + 8 c + 4 (L / 32)
    // + (L % 16) / 4, dims 32 dt + 16 ((L / 16) % 2) + 4 (L % 4) + [0, 4).
    const int tr_key = 4 * (lane >> 5) + ((lane & 15) >> 2);
    const int tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int dt = 0; dt < kD / 32; ++dt) {
          uint32_t w[4];
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int key = 32 * n + 16 * t + 8 * c + tr_key;
            const int dim = 32 * dt + tr_dim;
            const char* ptr = vt + swz(key, dim >> 3) + ((dim & 4) << 1);
            const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) v4s*)(ptr));
            w[2 * c] = uint32_t(uint16_t(r[0])) | (uint32_t(uint16_t(r[1])) << 16);
            w[2 * c + 1] = uint32_t(uint16_t(r[2])) | (uint32_t(uint16_t(r[3])) << 16);
          }
          o[dt] = mfma<kBf16>(make_uint4(w[0], w[1], w[2], w[3]), pk[n][t], o[dt]);
        }
  }

  // ---- normalise and store ------------------------------------------------
  // o[dt][r] is dim 32 dt + 8 (r / 4) + 4 half + r % 4 of query col.
  const float l_tot = l_run + swap_halves(l_run);
  if (!q_ok) return;
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;  // flash_attn.rs:66-71
  const int64_t orow = ((int64_t(q_begin) + qi) * a.n_heads + head) * kD;
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int dim = 32 * dt + 8 * g4 + 4 * half;
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = l_tot > 0.0f ? o[dt][4 * g4 + j] * inv : 0.0f;
      if (a.out_f32) {
        *reinterpret_cast<float4*>(static_cast<float*>(a.out) + orow + dim) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + orow + dim) =
            make_uint2(pack2<kBf16>(v[0], v[1]), pack2<kBf16>(v[2], v[3]));
      }
    }
}
}  // namespace

extern "C" int32_t it_paged_prefill(const it_kv_cache* c, const void* q, int32_t q_dtype, int32_t n_heads,
                                    const int32_t* cu_q, int32_t max_q_len, const int32_t* block_tables,
                                    int32_t max_blocks, const int32_t* ctx_lens, int32_t n_seqs, float scale,
                                    int32_t causal, void* out, int32_t out_dtype, void* stream) {
  const char* who = "it_paged_prefill";
  if (!c) return fail(IT_INVALID_INPUT, "%s: cache is NULL", who);
  if (c->dtype != IT_BF16 && c->dtype != IT_F16)
    return fail(IT_NOT_IMPLEMENTED, "%s: cache dtype %d (BF16 or F16 supported)", who, c->dtype);
  if (q_dtype != c->dtype) return fail(IT_NOT_IMPLEMENTED, "%s: q dtype %d must equal the cache dtype", who, q_dtype);
  if (out_dtype != IT_F32 && out_dtype != q_dtype)
    return fail(IT_NOT_IMPLEMENTED, "%s: out dtype must be F32 or the q dtype", who);
  if (c->head_dim != kD) return fail(IT_NOT_IMPLEMENTED, "%s: head_dim %d (128 supported)", who, c->head_dim);
  if (n_heads <= 0 || n_heads % c->n_kv_heads)
    return fail(IT_INVALID_INPUT, "%s: n_heads %d must be a positive multiple of n_kv_heads %d", who, n_heads,
                c->n_kv_heads);
  const int group = n_heads / c->n_kv_heads;
  if (group > kMaxGroup) return fail(IT_NOT_IMPLEMENTED, "%s: %d query heads per KV head (max %d)", who, group, kMaxGroup);
  if (n_seqs < 0 || n_seqs > 65535 || max_q_len < 0 || max_blocks <= 0)
    return fail(IT_INVALID_INPUT, "%s: n_seqs %d, max_q_len %d, max_blocks %d", who, n_seqs, max_q_len, max_blocks);
  if (n_seqs == 0 || max_q_len == 0) return IT_OK;
  if (!q || !cu_q || !block_tables || !ctx_lens || !out) return fail(IT_INVALID_INPUT, "%s: NULL tensor", who);
  if ((reinterpret_cast<uintptr_t>(q) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u))
    return fail(IT_INVALID_INPUT, "%s: q and out must be 16-byte aligned", who);
  if (!(scale == scale)) return fail(IT_INVALID_INPUT, "%s: scale is NaN", who);
  PrefillArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k_pool = static_cast<const char*>(c->k_pool);
  a.v_pool = static_cast<const char*>(c->v_pool);
  a.cu_q = cu_q;
  a.bt = block_tables;
  a.ctx_lens = ctx_lens;
  a.out = out;
  a.err = c->err_flag;
  a.page_bytes = c->page_bytes;
  a.num_blocks = c->num_blocks;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.n_heads = n_heads;
  a.n_kv_heads = c->n_kv_heads;
  a.group = group;
  a.max_blocks = max_blocks;
  a.log2_bs = c->log2_bs;
  a.causal = causal ? 1 : 0;
  a.out_f32 = out_dtype == IT_F32;
  int dev = -1;
  (void)hipGetDevice(&dev);
  if (dev != c->device) (void)hipSetDevice(c->device);
  const dim3 grid(unsigned((max_q_len + kQB - 1) / kQB), unsigned(c->n_kv_heads), unsigned(n_seqs));
  const size_t smem = 2 * kStageB;  // 64 KiB
  const dim3 block(unsigned(64 * group));
  const bool bf = c->dtype == IT_BF16;
  if (group <= 4) {
    if (bf) hipLaunchKernelGGL((paged_prefill_kernel<true, 4>), grid, block, smem, (hipStream_t)stream, a);
    else hipLaunchKernelGGL((paged_prefill_kernel<false, 4>), grid, block, smem, (hipStream_t)stream, a);
  } else {
    if (bf) hipLaunchKernelGGL((paged_prefill_kernel<true, kMaxGroup>), grid, block, smem, (hipStream_t)stream, a);
    else hipLaunchKernelGGL((paged_prefill_kernel<false, kMaxGroup>), grid, block, smem, (hipStream_t)stream, a);
  }
  hipError_t e = hipGetLastError();
  if (dev >= 0 && dev != c->device) (void)hipSetDevice(dev);
  if (e != hipSuccess) return fail(IT_DEVICE_ERROR, "%s: launch: %s", who, hipGetErrorString(e));
  return IT_OK;
}
