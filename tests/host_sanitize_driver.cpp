// Randomised exercise of the host allocator and slot manager (it_host.cpp),
// built with AddressSanitizer and UndefinedBehaviorSanitizer by
// test_host.py::test_host_code_under_sanitizers.  Every operation's
// outputs are checked against the pool's own counters:
//   - num_free + (distinct blocks some sequence holds) == capacity;
//   - every table entry is held (ref_count >= 1), and a block's ref_count is
//     the number of table entries naming it;
//   - each returned slot lies in the block the table names for its position,
//     and it_kv_manager_step's token sequence / position are that token's;
//   - the evicted list is exactly the blocks that went back to the pool:
//     every listed block is free afterwards, and every block some sequence
//     held before the step and none holds after it is listed (a block that
//     a fork still holds is never listed);
//   - release_seq with too small a capacity changes nothing;
//   - error paths (pool exhausted, table full, bad ids) return a status and
//     leave no memory error behind.
// Exit status 0 = all checks held; 1 = a check failed (message on stderr).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <random>
#include <vector>

#include "it_kv.h"

namespace {
long g_errors = 0, g_cows = 0, g_forks = 0, g_evicted = 0, g_ev_cap = 0, g_cow_cap = 0;

int fail(const char* what, long a = 0, long b = 0) {
  std::fprintf(stderr, "check failed: %s (%ld, %ld)\n", what, a, b);
  std::exit(1);
}

struct Ctx {
  it_block_pool* pool;
  it_kv_manager* mgr;
  int bs, seqs, mb;
};

// Tables, contexts and window starts, checked against the pool's counters.
void check_state(const Ctx& c) {
  std::vector<int32_t> t(size_t(c.seqs) * c.mb), ctx(c.seqs), st(c.seqs);
  if (it_kv_manager_tables(c.mgr, t.data(), c.mb, ctx.data(), st.data()) != IT_OK) fail("tables");
  std::map<int64_t, int64_t> refs;
  for (int s = 0; s < c.seqs; ++s) {
    if (st[s] < 0 || st[s] > ctx[s]) fail("window start", st[s], ctx[s]);
    for (int j = 0; j < c.mb; ++j) {
      const int32_t blk = t[size_t(s) * c.mb + j];
      if (blk < 0) continue;
      if (blk >= it_block_pool_capacity(c.pool)) fail("table entry range", blk);
      ++refs[blk];
    }
  }
  for (const auto& kv : refs)
    if (it_block_pool_ref_count(c.pool, kv.first) != kv.second)
      fail("ref count", kv.first, it_block_pool_ref_count(c.pool, kv.first));
  if (it_block_pool_num_free(c.pool) + int64_t(refs.size()) != it_block_pool_capacity(c.pool))
    fail("free + held != capacity", it_block_pool_num_free(c.pool), long(refs.size()));
}

// Blocks named by any table.
std::vector<char> held_blocks(const Ctx& c) {
  std::vector<int32_t> t(size_t(c.seqs) * c.mb);
  if (it_kv_manager_tables(c.mgr, t.data(), c.mb, nullptr, nullptr) != IT_OK) fail("tables");
  std::vector<char> h(size_t(it_block_pool_capacity(c.pool)), 0);
  for (int32_t b : t)
    if (b >= 0) h[size_t(b)] = 1;
  return h;
}

void check_evicted(const Ctx& c, const std::vector<char>& before, const int32_t* ev, int32_t n_ev) {
  const std::vector<char> after = held_blocks(c);
  std::vector<char> listed(before.size(), 0);
  for (int32_t i = 0; i < n_ev; ++i) {
    if (ev[i] < 0 || size_t(ev[i]) >= before.size()) fail("evicted id range", ev[i]);
    // Listed blocks went back to the pool; a LIFO hand-off in the same step
    // may have allocated one again (then it is held with refcount 1).
    if (!after[size_t(ev[i])] && it_block_pool_ref_count(c.pool, ev[i]) != 0) fail("evicted but held", ev[i]);
    listed[size_t(ev[i])] = 1;
  }
  for (size_t b = 0; b < before.size(); ++b)
    if (before[b] && !after[b] && !listed[b]) fail("freed but not listed", long(b));
}

void check_slots(const Ctx& c, const std::vector<int32_t>& seqs, const std::vector<int32_t>& ntok,
                 const std::vector<int32_t>& ctx_before, const std::vector<int64_t>& slots) {
  std::vector<int32_t> t(size_t(c.seqs) * c.mb);
  if (it_kv_manager_tables(c.mgr, t.data(), c.mb, nullptr, nullptr) != IT_OK) fail("tables");
  size_t k = 0;
  for (size_t i = 0; i < seqs.size(); ++i)
    for (int j = 0; j < ntok[i]; ++j, ++k) {
      const int64_t pos = int64_t(ctx_before[i]) + j;
      const int32_t blk = t[size_t(seqs[i]) * c.mb + pos / c.bs];
      if (blk < 0 || slots[k] != int64_t(blk) * c.bs + pos % c.bs) fail("slot", long(slots[k]), long(blk));
    }
}

int run(int window, uint32_t seed) {
  Ctx c{nullptr, nullptr, 16, 8, 64};
  const int64_t cap = 300;
  if (it_block_pool_new(cap, IT_BF16, &c.pool) != IT_OK) fail("pool");
  if (it_kv_manager_new(c.pool, c.bs, c.seqs, c.mb, window, &c.mgr) != IT_OK) fail("manager");
  std::mt19937 rng(seed);
  std::vector<int32_t> ev(4096), cs(64), cd(64);
  std::vector<int64_t> slots(4096);
  for (int step = 0; step < 3000; ++step) {
    const int op = int(rng() % 100);
    std::vector<int32_t> ctx(c.seqs);
    if (it_kv_manager_tables(c.mgr, nullptr, c.mb, ctx.data(), nullptr) != IT_OK) fail("ctx");
    if (op < 80) {  // append to a random subset, 1..40 tokens each
      std::vector<int32_t> seqs, ntok, before;
      for (int s = 0; s < c.seqs; ++s)
        if (rng() % 2) {
          seqs.push_back(s);
          ntok.push_back(1 + int(rng() % 40));
          before.push_back(ctx[s]);
        }
      if (seqs.empty()) continue;
      int32_t n_ev = 0, n_cow = 0;
      // Now and then the eviction and copy-on-write outputs are too small,
      // so their capacity errors are taken too.
      const int32_t ev_cap = (rng() % 6 == 0) ? int32_t(rng() % 3) : int32_t(ev.size());
      const int32_t cow_cap = (rng() % 6 == 0) ? int32_t(rng() % 2) : int32_t(cs.size());
      const std::vector<char> held_before = held_blocks(c);
      std::vector<int32_t> tseq(slots.size(), -7), tpos(slots.size(), -7), ctx_after(c.seqs, -7);
      const bool via_step = op >= 20 && op < 40;
      int32_t rc;
      if (op < 20) {
        rc = it_kv_manager_append(c.mgr, seqs.data(), ntok.data(), int32_t(seqs.size()), slots.data(), ev.data(),
                                  ev_cap, &n_ev);
      } else if (via_step) {
        it_kv_step_plan pl{};
        pl.slots = slots.data();
        pl.token_seq = tseq.data();
        pl.token_pos = tpos.data();
        pl.tokens_cap = int32_t(slots.size());
        pl.evicted = ev.data();
        pl.evicted_cap = ev_cap;
        pl.ctx_lens = ctx_after.data();
        rc = it_kv_manager_step(c.mgr, seqs.data(), ntok.data(), int32_t(seqs.size()), &pl);
        n_ev = pl.n_evicted;
      } else {
        rc = it_kv_manager_append_cow(c.mgr, seqs.data(), ntok.data(), int32_t(seqs.size()), slots.data(), ev.data(),
                                      ev_cap, &n_ev, cs.data(), cd.data(), cow_cap, &n_cow);
      }
      if (rc == IT_OK) {
        g_evicted += n_ev;
        check_evicted(c, held_before, ev.data(), n_ev);
      }
      if (rc == IT_OK && via_step) {
        size_t k = 0;
        for (size_t i = 0; i < seqs.size(); ++i)
          for (int j = 0; j < ntok[i]; ++j, ++k)
            if (tseq[k] != seqs[i] || tpos[k] != before[i] + j) fail("token seq/pos", tseq[k], tpos[k]);
        std::vector<int32_t> ctx_now(c.seqs);
        if (it_kv_manager_tables(c.mgr, nullptr, c.mb, ctx_now.data(), nullptr) != IT_OK) fail("ctx");
        if (ctx_now != ctx_after) fail("step ctx_lens");
      }
      if (rc != IT_OK) {
        ++g_errors;
        if (std::strstr(it_last_error(), "evicted capacity")) ++g_ev_cap;
        if (std::strstr(it_last_error(), "cow capacity")) ++g_cow_cap;
        // Whatever the error, no table names a freed block and no block is
        // lost: the counters hold before the recovery too.
        check_state(c);
        // Table full or pool exhausted: the state is unspecified, so start
        // every sequence over (releasing what each holds) and go on.
        for (int s = 0; s < c.seqs; ++s)
          if (it_kv_manager_release_seq(c.mgr, s, ev.data(), int32_t(ev.size()), &n_ev) != IT_OK)
            fail("release after error", s);
      } else {
        check_slots(c, seqs, ntok, before, slots);
        g_cows += n_cow;
        for (int i = 0; i < n_cow; ++i)
          if (cs[i] < 0 || cd[i] < 0 || cs[i] == cd[i]) fail("cow pair", cs[i], cd[i]);
      }
    } else if (op < 90) {  // release one sequence
      int32_t n_ev = 0;
      const int32_t s = int32_t(rng() % c.seqs);
      const std::vector<char> held_before = held_blocks(c);
      if (ctx[s] > 0) {
        // Too small a capacity: an error, and nothing changes.
        std::vector<int32_t> t0(size_t(c.seqs) * c.mb), t1(size_t(c.seqs) * c.mb);
        it_kv_manager_tables(c.mgr, t0.data(), c.mb, nullptr, nullptr);
        const int64_t free0 = it_block_pool_num_free(c.pool);
        if (it_kv_manager_release_seq(c.mgr, s, ev.data(), 0, &n_ev) == IT_OK) fail("release cap 0 accepted", s);
        it_kv_manager_tables(c.mgr, t1.data(), c.mb, nullptr, nullptr);
        if (t0 != t1 || it_block_pool_num_free(c.pool) != free0) fail("release error changed state", s);
      }
      if (it_kv_manager_release_seq(c.mgr, s, ev.data(), int32_t(ev.size()), &n_ev) != IT_OK) fail("release");
      check_evicted(c, held_before, ev.data(), n_ev);
    } else {  // fork into an empty sequence, if there is one
      int dst = -1;
      for (int s = 0; s < c.seqs; ++s)
        if (ctx[s] == 0) dst = s;
      const int src = int(rng() % c.seqs);
      if (dst >= 0 && src != dst) {
        if (it_kv_manager_fork(c.mgr, src, dst) != IT_OK) fail("fork", src, dst);
        ++g_forks;
      }
    }
    check_state(c);
  }
  // Bad ids and arguments: statuses, never memory errors.
  int32_t n_ev = 0;
  if (it_kv_manager_release_seq(c.mgr, c.seqs, ev.data(), 4, &n_ev) == IT_OK) fail("release out of range");
  if (it_block_pool_free(c.pool, cap) == IT_OK) fail("free out of range");
  if (it_block_pool_share(c.pool, -1) == IT_OK) fail("share out of range");
  it_kv_manager_destroy(c.mgr);
  it_block_pool_destroy(c.pool);
  return 0;
}
}  // namespace

// The case of a window eviction past evicted_cap: bs 16, window 16, 31
// tokens, then one more with no room for the freed id.  The call fails, the
// table no longer names the block, and releasing the sequence afterwards
// frees nothing twice (another sequence's block stays allocated).
void evict_capacity_case() {
  it_block_pool* pool = nullptr;
  it_kv_manager* mgr = nullptr;
  if (it_block_pool_new(8, IT_BF16, &pool) != IT_OK || it_kv_manager_new(pool, 16, 2, 4, 16, &mgr) != IT_OK)
    fail("evict case setup");
  Ctx c{pool, mgr, 16, 2, 4};
  std::vector<int64_t> slots(64);
  std::vector<int32_t> ev(8);
  int32_t seq = 0, n = 31, n_ev = 0;
  if (it_kv_manager_append(mgr, &seq, &n, 1, slots.data(), ev.data(), 8, &n_ev) != IT_OK) fail("evict case 31");
  n = 1;
  if (it_kv_manager_append(mgr, &seq, &n, 1, slots.data(), ev.data(), 0, &n_ev) == IT_OK) fail("evict cap 0 accepted");
  check_state(c);
  seq = 1;
  n = 20;
  if (it_kv_manager_append(mgr, &seq, &n, 1, slots.data(), ev.data(), 8, &n_ev) != IT_OK) fail("evict case seq 1");
  if (it_kv_manager_release_seq(mgr, 0, ev.data(), 8, &n_ev) != IT_OK) fail("evict case release");
  check_state(c);
  // Copy-on-write with no room for the pair: no block leaks.
  if (it_kv_manager_fork(mgr, 1, 0) != IT_OK) fail("cow case fork");
  int32_t cs = -1, cd = -1, n_cow = 0;
  seq = 0;
  n = 1;
  if (it_kv_manager_append_cow(mgr, &seq, &n, 1, slots.data(), ev.data(), 8, &n_ev, &cs, &cd, 0, &n_cow) == IT_OK)
    fail("cow cap 0 accepted");
  check_state(c);
  for (int s = 0; s < 2; ++s)
    if (it_kv_manager_release_seq(mgr, s, ev.data(), 8, &n_ev) != IT_OK) fail("cow case release", s);
  if (it_block_pool_num_free(pool) != 8) fail("blocks lost", long(it_block_pool_num_free(pool)));
  it_kv_manager_destroy(mgr);
  it_block_pool_destroy(pool);
}

int main() {
  evict_capacity_case();
  for (uint32_t seed = 1; seed <= 4; ++seed) {
    run(0, seed);
    run(100, seed);
  }
  std::printf("host sanitize driver: ok (%ld error recoveries, %ld of them evicted capacity, %ld cow capacity; "
              "%ld forks, %ld copy-on-write pairs, %ld evictions)\n",
              g_errors, g_ev_cap, g_cow_cap, g_forks, g_cows, g_evicted);
  // Each path must have been taken, or the run proves little.
  if (!g_errors || !g_ev_cap || !g_cow_cap || !g_forks || !g_cows || !g_evicted) return 1;
  return 0;
}
