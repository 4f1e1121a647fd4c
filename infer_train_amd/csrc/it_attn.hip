// it_attn.hip -- C ABI of the attention entry points: paged split-K decode
// (+ combine) and the Backend FlashAttention operator over contiguous K/V.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>

#include "it_decode.hpp"
#include "it_decode_launch.hpp"
#include "it_internal.hpp"

using namespace itkv;

namespace {
constexpr int kMaxParts = 4096;
constexpr int kCompactSeqs = 512;

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct WsLayout {
  size_t o_bytes, ml_bytes, total;
};
WsLayout ws_layout(int64_t n_seqs, int64_t n_heads, int64_t head_dim, int64_t max_parts) {
  WsLayout w;
  w.o_bytes = align_up(size_t(n_seqs * n_heads * max_parts * head_dim) * 4, 256);
  w.ml_bytes = align_up(size_t(n_seqs * n_heads * max_parts) * 8, 256);
  w.total = w.o_bytes + w.ml_bytes;
  return w;
}

int pick_chunk(int group) {
  for (int g = 8; g >= 1; --g)
    if (group % g == 0) return g;
  return 1;
}

hipError_t launch_split(int32_t dt, int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  switch (dt) {
    case IT_BF16: return launch_decode_bf16(d, gc, a, grid, s);
    case IT_F16: return launch_decode_f16(d, gc, a, grid, s);
    case IT_F32: return launch_decode_f32(d, gc, a, grid, s);
    case IT_Q8_0: return launch_decode_q8_0(d, gc, a, grid, s);
    case IT_Q4_0: return launch_decode_q4_0(d, gc, a, grid, s);
    case IT_Q4_1: return launch_decode_q4_1(d, gc, a, grid, s);
    case IT_Q5_0: return launch_decode_q5_0(d, gc, a, grid, s);
    case IT_Q5_1: return launch_decode_q5_1(d, gc, a, grid, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_combine(int d, const DecodeArgs& a, int n_seqs, void* out, int32_t out_dtype, hipStream_t s) {
  // One workgroup per (row, 128-dim slice), rows placed on the XCD whose
  // split workgroups wrote them (CombineMap): grid.x = 8 * the largest XCD
  // range.
  CombineMap map;
  map.gc = a.group / a.chunks;
  map.max_parts = a.max_parts;
  map.n_rows = int64_t(n_seqs) * a.n_heads;
  map.q8 = (int64_t(n_seqs) * a.n_kv_heads * a.chunks * a.max_parts + 7) / 8;
  int64_t widest = 0;
  for (int x = 0; x < 8; ++x) widest = std::max(widest, map.first_row(x + 1) - map.first_row(x));
  const dim3 grid(unsigned(8 * widest), 1u, unsigned(d / 128));
  // Rows of more than 32 partitions (one wave's batch) take four waves.
  const bool wide = map.max_parts > 32;
#define IT_COMBINE(DD, NWW)                                                                                       \
  hipLaunchKernelGGL((paged_decode_combine<DD, NWW>), grid, dim3(64 * NWW), 0, s, a.ws_o, a.ws_ml, map.q8,          \
                     map.n_rows, map.gc, map.max_parts, a.n_heads, a.ctx_lens, a.start_pos, a.ctx_const, a.partition, \
                     out, out_dtype)
  if (d == 128) {
    if (wide) IT_COMBINE(128, 4);
    else IT_COMBINE(128, 1);
  } else if (d == 256) {
    if (wide) IT_COMBINE(256, 4);
    else IT_COMBINE(256, 1);
  } else {
    return hipErrorInvalidValue;
  }
#undef IT_COMBINE
  return hipGetLastError();
}

// Shared driver of it_paged_decode and it_flash_attention.
// phases: 1 = split pass, 2 = combine pass, 3 = both.
int32_t run_decode(const char* who, int32_t cache_dt, int32_t q_dtype, int32_t out_dtype, int d,
                   int n_seqs, int max_tokens, DecodeArgs a, void* ws, size_t ws_bytes, void* out,
                   hipStream_t s, int phases = 3) {
  const int32_t want_q = (cache_dt == IT_BF16 || cache_dt == IT_F16) ? cache_dt : IT_F32;
  if (q_dtype != want_q)
    return fail(IT_NOT_IMPLEMENTED, "%s: cache dtype %d takes q dtype %d, got %d", who, cache_dt, want_q, q_dtype);
  if (out_dtype != IT_F32 && out_dtype != q_dtype)
    return fail(IT_NOT_IMPLEMENTED, "%s: out dtype must be F32 or the q dtype", who);
  if (d != 128 && d != 256) return fail(IT_NOT_IMPLEMENTED, "%s: head_dim %d (128 or 256 supported)", who, d);
  if (a.log2_bs < 3) return fail(IT_NOT_IMPLEMENTED, "%s: block_size must be >= 8", who);
  if (a.partition < 64 || a.partition > 2048 || a.partition % 64)
    return fail(IT_INVALID_INPUT, "%s: partition %d must be a multiple of 64 in [64, 2048]", who, a.partition);
  if (n_seqs <= 0 || n_seqs > 65535) return fail(IT_INVALID_INPUT, "%s: n_seqs %d outside [1, 65535]", who, n_seqs);
  if (max_tokens < 0) return fail(IT_INVALID_INPUT, "%s: max_tokens %d < 0", who, max_tokens);
  if (a.n_heads <= 0 || a.n_heads % a.n_kv_heads)
    return fail(IT_INVALID_INPUT, "%s: n_heads %d must be a positive multiple of n_kv_heads %d", who, a.n_heads,
                a.n_kv_heads);
  if (!a.q || !out || !ws) return fail(IT_INVALID_INPUT, "%s: NULL tensor", who);
  if (reinterpret_cast<uintptr_t>(out) & (out_dtype == IT_F32 ? 7u : 3u))
    return fail(IT_INVALID_INPUT, "%s: out must be %d-byte aligned", who, out_dtype == IT_F32 ? 8 : 4);
  if ((reinterpret_cast<uintptr_t>(a.q) & 15u) || (reinterpret_cast<uintptr_t>(ws) & 255u))
    return fail(IT_INVALID_INPUT, "%s: q must be 16-byte and ws 256-byte aligned", who);
  a.max_parts = max_tokens > 0 ? (max_tokens + a.partition - 1) / a.partition : 1;
  if (a.max_parts > kMaxParts) return fail(IT_INVALID_INPUT, "%s: %d partitions > %d", who, a.max_parts, kMaxParts);
  const WsLayout w = ws_layout(n_seqs, a.n_heads, d, a.max_parts);
  if (ws_bytes < w.total) return fail(IT_INVALID_INPUT, "%s: workspace %zu < %zu bytes", who, ws_bytes, w.total);
  a.ws_o = static_cast<float*>(ws);
  a.ws_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + w.o_bytes);
  a.group = a.n_heads / a.n_kv_heads;
  const int gc = pick_chunk(a.group);
  a.chunks = a.group / gc;
  if (int64_t(a.n_kv_heads) * a.chunks > 65535) return fail(IT_NOT_IMPLEMENTED, "%s: too many head chunks", who);
  a.max_pages = (a.partition >> a.log2_bs) + 2;
  a.n_seqs = n_seqs;
  const int64_t n_units = int64_t(a.max_parts) * a.n_kv_heads * a.chunks * n_seqs;
  // Per-sequence contexts: a one-dimensional grid over the non-empty units
  // (every wave scans the n_seqs context lengths, so only up to 512), a
  // multiple of 8 workgroups so that every XCD's range of units is covered.
  a.compact = (a.ctx_lens != nullptr && n_seqs <= kCompactSeqs && n_units < (int64_t(1) << 30)) ? 1 : 0;
  const int64_t n_wg = a.compact ? (n_units + 7) / 8 * 8 : n_units;
  const size_t smem = decode_smem_bytes(cache_dt, gc, d, a.partition, a.max_pages, n_wg);
  if (smem > kMaxDecodeLds) return fail(IT_INVALID_INPUT, "%s: partition %d needs %zu bytes of LDS", who, a.partition, smem);
  if (max_tokens > 0 && (phases & 1)) {
    const dim3 grid = a.compact ? dim3(unsigned(n_wg), 1u, 1u)
                                : dim3(unsigned(a.max_parts), unsigned(a.n_kv_heads * a.chunks), unsigned(n_seqs));
    hipError_t e = launch_split(cache_dt, d, gc, a, grid, s);
    if (e != hipSuccess) return fail(IT_DEVICE_ERROR, "%s: split launch: %s", who, hipGetErrorString(e));
  }
  if (phases & 2) {
    hipError_t e = launch_combine(d, a, n_seqs, out, out_dtype, s);
    if (e != hipSuccess) return fail(IT_DEVICE_ERROR, "%s: combine launch: %s", who, hipGetErrorString(e));
  }
  return IT_OK;
}
}  // namespace

extern "C" size_t it_paged_decode_workspace(int32_t n_seqs, int32_t n_heads, int32_t head_dim,
                                            int32_t max_tokens, int32_t partition) {
  if (n_seqs <= 0 || n_heads <= 0 || head_dim <= 0 || partition <= 0 || max_tokens < 0) return 0;
  const int64_t parts = max_tokens > 0 ? (int64_t(max_tokens) + partition - 1) / partition : 1;
  return ws_layout(n_seqs, n_heads, head_dim, parts).total;
}

extern "C" int32_t it_paged_decode_partition(int32_t dtype, int32_t head_dim, int32_t block_size, int32_t n_heads,
                                             int32_t n_kv_heads, const int32_t* ctx_lens, const int32_t* start_pos,
                                             int32_t n_seqs, int32_t n_cu, int32_t* partition) {
  constexpr const char* who = "it_paged_decode_partition";
  if (!ctx_lens || !partition) return fail(IT_INVALID_INPUT, "%s: NULL argument", who);
  if (n_seqs <= 0) return fail(IT_INVALID_INPUT, "%s: n_seqs %d <= 0", who, n_seqs);
  if (n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads)
    return fail(IT_INVALID_INPUT, "%s: n_heads %d must be a positive multiple of n_kv_heads %d", who, n_heads,
                n_kv_heads);
  if (block_size < 8 || (block_size & (block_size - 1)))
    return fail(IT_INVALID_INPUT, "%s: block_size %d must be a power of two >= 8", who, block_size);
  if (head_dim != 128 && head_dim != 256) return fail(IT_NOT_IMPLEMENTED, "%s: head_dim %d", who, head_dim);
  if (n_cu <= 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
      return fail(IT_DEVICE_ERROR, "%s: cannot read the device's compute-unit count", who);
  }
  int log2_bs = 0;
  while ((1 << log2_bs) < block_size) ++log2_bs;
  const int group = n_heads / n_kv_heads, gc = pick_chunk(group);
  const int64_t hc = int64_t(n_kv_heads) * (group / gc);
  int64_t max_n = 0;
  for (int b = 0; b < n_seqs; ++b) {
    const int64_t n = int64_t(ctx_lens[b]) - (start_pos ? start_pos[b] : 0);
    if (n > max_n) max_n = n;
  }
  // Resident slots of one round: four workgroups per compute unit, fewer
  // where the LDS does not hold four.
  int best = 0, longest_two = 0;
  int64_t best_rounds = 0;
  for (int p = 64; p <= 2048; p += 64) {
    const int64_t parts = max_n > 0 ? (max_n + p - 1) / p : 1;
    if (parts > kMaxParts) continue;
    const size_t smem =
        decode_smem_bytes(dtype, gc, head_dim, p, (p >> log2_bs) + 2, parts * hc * n_seqs);
    if (smem > kMaxDecodeLds) continue;
    const int64_t per_cu = std::min<int64_t>(4, int64_t(kMaxDecodeLds / smem));
    int64_t units = 0;
    for (int b = 0; b < n_seqs; ++b) {
      const int64_t n = int64_t(ctx_lens[b]) - (start_pos ? start_pos[b] : 0);
      if (n > 0) units += (n + p - 1) / p;
    }
    const int64_t rounds = (units * hc + per_cu * n_cu - 1) / (per_cu * n_cu);
    if (!best || rounds < best_rounds) {
      best = p;
      best_rounds = rounds;
    }
    if (per_cu >= 2) longest_two = p;
  }
  if (!best) return fail(IT_NOT_IMPLEMENTED, "%s: no partition fits (max context %lld)", who, (long long)max_n);
  // Beyond two rounds the workgroups stream back to back and the machine
  // stays full whatever the size: then the longest partition that still
  // keeps two workgroups per CU writes the fewest partials and starts the
  // fewest workgroups.
  *partition = (best_rounds > 2 && longest_two) ? longest_two : best;
  return IT_OK;
}

namespace {
int32_t paged_decode_phases(const char* who, const it_kv_cache* c, const void* q, int32_t q_dtype,
                            int32_t n_heads, const int32_t* block_tables, int32_t max_blocks,
                            const int32_t* ctx_lens, const int32_t* start_pos, int32_t n_seqs,
                            int32_t max_tokens, float scale, int32_t partition, void* ws, size_t ws_bytes,
                            void* out, int32_t out_dtype, void* stream, int phases) {
  if (!c) return fail(IT_INVALID_INPUT, "%s: cache is NULL", who);
  if (int32_t rc = one_layer(c, who)) return rc;
  if (!block_tables || !ctx_lens) return fail(IT_INVALID_INPUT, "%s: NULL block_tables/ctx_lens", who);
  if (max_blocks <= 0) return fail(IT_INVALID_INPUT, "%s: max_blocks %d", who, max_blocks);
  if (!(scale == scale)) return fail(IT_INVALID_INPUT, "%s: scale is NaN", who);
  DecodeArgs a{};
  a.q = q;
  a.k_pool = static_cast<const char*>(c->k_pool);
  a.v_pool = static_cast<const char*>(c->v_pool);
  a.bt = block_tables;
  a.ctx_lens = ctx_lens;
  a.start_pos = start_pos;
  a.mask = nullptr;
  a.err = c->err_flag;
  a.page_bytes = c->page_bytes;
  a.num_blocks = c->num_blocks;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.ctx_const = 0;
  a.max_blocks = max_blocks;
  a.n_heads = n_heads;
  a.n_kv_heads = c->n_kv_heads;
  a.log2_bs = c->log2_bs;
  a.partition = partition;
  int dev = -1;
  (void)hipGetDevice(&dev);
  if (dev != c->device) (void)hipSetDevice(c->device);
  int32_t rc = run_decode(who, c->dtype, q_dtype, out_dtype, c->head_dim, n_seqs, max_tokens, a, ws, ws_bytes, out,
                          (hipStream_t)stream, phases);
  if (dev >= 0 && dev != c->device) (void)hipSetDevice(dev);
  return rc;
}
}  // namespace

#define IT_DECODE_ARGS                                                                                          \
  const it_kv_cache *c, const void *q, int32_t q_dtype, int32_t n_heads, const int32_t *block_tables,          \
      int32_t max_blocks, const int32_t *ctx_lens, const int32_t *start_pos, int32_t n_seqs, int32_t max_tokens, \
      float scale, int32_t partition, void *ws, size_t ws_bytes, void *out, int32_t out_dtype, void *stream
#define IT_DECODE_PASS \
  c, q, q_dtype, n_heads, block_tables, max_blocks, ctx_lens, start_pos, n_seqs, max_tokens, scale, partition, ws, \
      ws_bytes, out, out_dtype, stream

extern "C" int32_t it_paged_decode(IT_DECODE_ARGS) {
  return paged_decode_phases("it_paged_decode", IT_DECODE_PASS, 3);
}
extern "C" int32_t it_paged_decode_split(IT_DECODE_ARGS) {
  return paged_decode_phases("it_paged_decode_split", IT_DECODE_PASS, 1);
}
extern "C" int32_t it_paged_decode_combine(IT_DECODE_ARGS) {
  return paged_decode_phases("it_paged_decode_combine", IT_DECODE_PASS, 2);
}

// ---- it_paged_decode_noalloc: the decode without a caller workspace ------
// For callers that cannot allocate (code under HIP graph capture, serving
// loops, harnesses that forbid hipMalloc): the (m, l, O) partials live in
// `scratch`, a file-scope device array of kNoAllocScratch bytes that every
// GPU the library runs on holds until the process ends.  In host code the
// array's name is only a host-side stand-in, so its device address is
// looked up once per device (hipGetSymbolAddress, with that device current)
// and only that address is used.  Calls on one GPU share the array: calls
// that overlap in time on one GPU (two streams) race.
namespace {
constexpr size_t kNoAllocScratch = size_t(32) << 20;  // 32 MiB
constexpr int kMaxDevices = 64;
static __device__ __align__(256) char scratch[kNoAllocScratch];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on `device` (current), or NULL with the
// thread's message set.  it_kv_cache_new / _wrap look it up for the
// cache's device already (noalloc_prepare), so a call made under graph
// capture finds it here without a runtime call.
void* scratch_address(int device) {
  if (device < 0 || device >= kMaxDevices) {
    fail(IT_DEVICE_ERROR, "it_paged_decode_noalloc: device %d outside [0, %d)", device, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      fail(IT_DEVICE_ERROR, "it_paged_decode_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[device] = ptr;
  }
  return g_scratch_ptr[device];
}
}  // namespace

int32_t itkv::noalloc_prepare(int device) { return scratch_address(device) ? IT_OK : IT_DEVICE_ERROR; }

extern "C" int32_t it_paged_decode_noalloc(const it_kv_cache* c, const void* q, int32_t q_dtype, int32_t n_heads,
                                           const int32_t* block_tables, int32_t max_blocks, const int32_t* ctx_lens,
                                           const int32_t* start_pos, int32_t n_seqs, int32_t max_tokens, float scale,
                                           int32_t partition, void* out, int32_t out_dtype, void* stream) {
  constexpr const char* who = "it_paged_decode_noalloc";
  if (!c) return fail(IT_INVALID_INPUT, "%s: cache is NULL", who);
  const size_t need = it_paged_decode_workspace(n_seqs, n_heads, c->head_dim, max_tokens, partition);
  if (need == 0) return fail(IT_INVALID_INPUT, "%s: invalid sizes", who);
  if (need > kNoAllocScratch)
    return fail(IT_INVALID_INPUT, "%s: the partials need %zu bytes, more than the %zu-byte scratch (fewer sequences, "
                "fewer heads or longer partitions fit)", who, need, kNoAllocScratch);
  int dev = -1;
  (void)hipGetDevice(&dev);
  if (dev != c->device) (void)hipSetDevice(c->device);
  void* ws = scratch_address(c->device);
  if (dev >= 0 && dev != c->device) (void)hipSetDevice(dev);
  if (!ws) return IT_DEVICE_ERROR;
  return paged_decode_phases(who, c, q, q_dtype, n_heads, block_tables, max_blocks, ctx_lens, start_pos, n_seqs,
                             max_tokens, scale, partition, ws, kNoAllocScratch, out, out_dtype, stream, 3);
}

// The Backend FlashAttention operator (src/backend/arm.rs:304-370) runs the
// same kernels: contiguous K/V [n_kv][D] are pages of 16 rows under the
// identity block table, one KV head shared by all n_heads query heads.
// The partition grows with the key count: one query's keys are spread over
// up to 16 partitions (64..512 tokens each), so a short context still
// streams through many workgroups instead of one long chain of loads.
namespace {
constexpr int kFaBlock = 16;
int fa_partition(int32_t n_kv) {
  const int per = (n_kv + 15) / 16;
  const int p = (per + 63) / 64 * 64;
  return p < 64 ? 64 : (p > 512 ? 512 : p);
}
}  // namespace

extern "C" size_t it_flash_attention_workspace(int32_t n_heads, int32_t head_dim, int32_t n_kv) {
  // Plus 256 bytes for the device error word.
  return it_paged_decode_workspace(1, n_heads, head_dim, n_kv, fa_partition(n_kv)) + 256;
}

extern "C" int32_t it_flash_attention(const float* q, const float* k, const float* v, const float* mask,
                                      float* out, int32_t n_heads, int32_t head_dim, int32_t n_kv, void* ws,
                                      size_t ws_bytes, void* stream) {
  if (!q || !k || !v || !out || !ws) return fail(IT_INVALID_INPUT, "it_flash_attention: NULL tensor");
  if (n_heads <= 0 || head_dim <= 0 || n_kv < 0)
    return fail(IT_INVALID_INPUT, "it_flash_attention: n_heads=%d head_dim=%d n_kv=%d", n_heads, head_dim, n_kv);
  if ((reinterpret_cast<uintptr_t>(k) & 15u) || (reinterpret_cast<uintptr_t>(v) & 15u))
    return fail(IT_INVALID_INPUT, "it_flash_attention: k/v must be 16-byte aligned");
  const size_t need = it_flash_attention_workspace(n_heads, head_dim, n_kv);
  if (ws_bytes < need) return fail(IT_INVALID_INPUT, "it_flash_attention: workspace %zu < %zu bytes", ws_bytes, need);
  DecodeArgs a{};
  a.q = q;
  a.k_pool = reinterpret_cast<const char*>(k);
  a.v_pool = reinterpret_cast<const char*>(v);
  a.bt = nullptr;
  a.ctx_lens = nullptr;
  a.start_pos = nullptr;
  a.mask = mask;
  a.err = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + need - 256);
  a.page_bytes = int64_t(kFaBlock) * head_dim * 4;
  a.num_blocks = (int64_t(n_kv) + kFaBlock - 1) / kFaBlock;
  if (a.num_blocks == 0) a.num_blocks = 1;
  const float scale = 1.0f / sqrtf(float(head_dim));  // arm.rs:367
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.ctx_const = n_kv;
  a.max_blocks = int32_t(a.num_blocks);
  a.n_heads = n_heads;
  a.n_kv_heads = 1;
  a.log2_bs = 4;
  a.partition = fa_partition(n_kv);
  return run_decode("it_flash_attention", IT_F32, IT_F32, IT_F32, head_dim, 1, n_kv, a, ws, need - 256, out,
                    (hipStream_t)stream);
}

extern "C" int32_t it_paged_prefill(const it_kv_cache* c, const void* q, int32_t q_dtype, int32_t n_heads,
                                    const int32_t* cu_q, int32_t max_q_len, const int32_t* block_tables,
                                    int32_t max_blocks, const int32_t* ctx_lens, int32_t n_seqs, float scale,
                                    int32_t causal, void* out, int32_t out_dtype, void* stream);
