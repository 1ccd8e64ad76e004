// Device-side LRU expert cache for gfx950 (MI355X): the manager, the fused manager +
// moe_align_block_size, and the miss gather.
//
// Semantics are those of kernels/lru/r4d_lru.hip (lru_manage_k :187-269, pickVictims :119-185,
// lru_fused_k :418-575, lru_gather_k :271-301); the entry points at the bottom keep its C-ABI.
// The implementation is this build's own, shaped for wave64 CDNA4:
//
//  * One workgroup of 256 threads (one wave per SIMD), six barriers for the fused kernel at
//    decode sizes (three for the manager). Every global load is issued up front, so the kernel
//    pays one memory round trip, not one per phase. Decode-sized align outputs are built in
//    LDS and written once, coalesced, with the sentinels past num_post_pad written directly;
//    larger ones are pre-filled with their sentinels in global memory, and only the first
//    barrier waits for global stores (the rest order LDS only).
//  * Cross-lane reductions and scans are DPP + v_readlane (wave-uniform scalars), not LDS
//    shuffles.
//  * Routed / non-resident sets are 64-bit-word bitmaps built from wave ballots; misses are
//    ranked in ascending expert id by popcount prefixes (no block scan).
//  * Victims -- the nins smallest (stamp << 20 | slot) keys among slots whose expert is not
//    routed, ascending -- are chosen by ONE wave with no barrier: a radix search for the
//    boundary stamp (8-bit digits counted in an LDS histogram, or one ballot + popcount per slot
//    register per key bit for stamps past 32 bits), a ballot compaction of the keys at or below
//    it, and a rank of the <= nins survivors among themselves. Cost grows with key bits and nins, never with a per-insert block reduction,
//    so there is no insert-count cliff.
//  * Align is stable at every mk: a token's rank inside its bucket is the number of earlier
//    tokens routed to the same expert -- up to 256 tokens a popcount of the expert's token
//    bitmap below it (each token places itself), above that a bit-sliced wave match plus
//    per-wave counts in LDS. Above 1536 tokens the sorted arrays are written by place_k, one
//    1024-thread workgroup per 1024 tokens, each counting the tokens before its own.
//
// Preconditions (checked by the reference's own tests after every step, tests/lru/test_lru.py:
// 138-145): table/map_cold complementary, table[slot_expert[s]] == s for resident slots,
// entries in range. Under them the results equal the reference kernel's bit for bit.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "quant_row.h"
#include "rlu.h"
#include "wave.h"

namespace rlu {

constexpr int NT = 256;
constexpr int NW = NT / WAVE;
constexpr int MAXS = 1024;
constexpr int MAXE = 1024;
constexpr int MAXINS = 1024;
constexpr int SLOT_BITS = 20;
constexpr int QS = MAXS / WAVE;      // slot registers per lane in the selecting wave
constexpr int EJ = MAXE / NT;        // experts per thread
constexpr int NWORD = MAXE / 64;     // bitmap words

constexpr int MLOADS = 32;           // id loads in flight per thread when marking > NT tokens
constexpr int TW = NT / 64;          // u64 words of a per-expert token mask (<= NT tokens)
constexpr int LSTAGE = 4096;         // align outputs staged in LDS up to this many sorted ids
constexpr int NBSTAGE = 256;         // ... and this many expert ids, per side

struct LruLds {
  uint64_t rbits[NWORD];             // routed this step (by expert)
  uint64_t nres[NWORD];              // table[e] < 0 on entry (by expert)
  uint64_t sbusy[NWORD];             // the slot's expert is routed this step (by slot)
  int mpre[NWORD];                   // misses in earlier bitmap words
  int misc[4];                       // nact, nins
  int tab[MAXE];                     // table on entry
  int ecnt[MAXE];                    // general path: tokens per expert, then the per-expert
                                     // base of the token chunk being placed
  int vslot[MAXINS];                 // victim slot of rank r
  int vold[MAXINS];                  // expert evicted from it (or -1)
  int vrank[MAXS];                   // align: the rank of the miss a slot takes this step, or -1
  int vcnt[MAXINS];                  // align: tokens of the miss of rank r < nact
  int vexp[MAXINS];                  // align: the miss of rank r < nins (ascending expert id)
  int mpw[NW][NWORD];                // align: each wave's own copy of the miss prefix (mpre)
  alignas(16) uint64_t vkey[MAXINS]; // victims, compacted, before ranking
  alignas(16) int hist[256];         // the victim search's digit histogram
  int vpack[MAXINS];                 // (slot << 16) | (old expert & 0xffff), same order
  int cnt_h[MAXS];                   // post-update tokens per hot bucket (slot)
  int cnt_c[MAXE];                   // post-update tokens per cold bucket (expert)
  int cum_h[MAXS];
  int cum_c[MAXE];
  int wsum[NW][2];
  union {
    uint64_t tmask[MAXE][TW];        // staged path: bit i of expert e = token i routes to e
    uint8_t wcnt[NW][MAXE];          // general path: tokens per (wave, expert) in a chunk
  } tk;
  alignas(16) int stage_h[LSTAGE];   // 16-byte units for the fill and the copy-out
  alignas(16) int stage_c[LSTAGE];
  int stage_eh[NBSTAGE], stage_ec[NBSTAGE];
};

// cnt[e] += the number of ids[lo, hi) equal to e, for e in [0, E), with VL 16-byte loads in
// flight per thread (ids + lo 16-byte aligned, hi - lo a multiple of 4). Counts are LDS
// atomics, so the order of the tokens does not matter.
constexpr int VL = 16;
__device__ __forceinline__ void count_ids_vec(const int* __restrict__ ids, int lo, int hi, int E,
                                              int* cnt) {
  const int4* v = reinterpret_cast<const int4*>(ids + lo);
  const int nv = (hi - lo) / 4;
  for (int j = threadIdx.x; j < nv; j += VL * NT) {
    int4 a[VL];
#pragma unroll
    for (int u = 0; u < VL; ++u) a[u] = v[min(j + u * NT, nv - 1)];
#pragma unroll
    for (int u = 0; u < VL; ++u) {
      if (j + u * NT < nv) {
        if ((unsigned)a[u].x < (unsigned)E) atomicAdd(&cnt[a[u].x], 1);
        if ((unsigned)a[u].y < (unsigned)E) atomicAdd(&cnt[a[u].y], 1);
        if ((unsigned)a[u].z < (unsigned)E) atomicAdd(&cnt[a[u].z], 1);
        if ((unsigned)a[u].w < (unsigned)E) atomicAdd(&cnt[a[u].w], 1);
      }
    }
  }
}

__device__ __forceinline__ bool bit_of(const uint64_t* bm, int e) {
  return ((bm[e >> 6] >> (e & 63)) & 1ull) != 0;
}

// ---- victim selection (one wave) ------------------------------------------------------
// Victims are the nact smallest (stamp, slot) pairs among evictable slots, ascending; rank r
// installs miss r. Stamps are split into the oldest group (stamp == smin) and the rest:
//   * if the oldest group alone has >= nact slots (always at nact == 1, and the usual case
//     in steady state, where a whole step's hits share one stamp), the victims are its first
//     nact slots in slot order -- no search, no ranking;
//   * otherwise a search over the stamp range, 8 bits per pass, finds the boundary stamp tau
//     (#{stamp < tau} < nact <= #{stamp <= tau}); the boundary group is cut in slot order by
//     ballot prefix, and the <= nact survivors are ranked among themselves.
// Stamps outside [0, 2^43) fall back to a search over the reference key (stamp << 20) | slot
// itself (biased to unsigned order), which the reference defines with wrap-around.

// writes victim of rank p
__device__ __forceinline__ void put_victim(LruLds& L, int p, int slot, int old) {
  L.vslot[p] = slot;
  L.vold[p] = old;
  L.vrank[slot] = p;
}

// rank the n compacted keys L.vkey[0..n) among themselves (keys unique), then install
__device__ __forceinline__ void rank_compacted(LruLds& L, int n) {
  wave_lds_sync();
  const int lane = lane_id();
  for (int p = lane; p < n; p += WAVE) {
    const uint64_t v = L.vkey[p];
    int r = 0;
    int j = 0;
    for (; j + 4 <= n; j += 4)
      r += (L.vkey[j] < v) + (L.vkey[j + 1] < v) + (L.vkey[j + 2] < v) + (L.vkey[j + 3] < v);
    for (; j < n; ++j) r += (L.vkey[j] < v);
    const int pk = L.vpack[p];
    put_victim(L, r, pk >> 16, (int)(short)(pk & 0xffff));
  }
}

template <int Q>
__device__ __forceinline__ void compact_victims(LruLds& L, const bool* vic, const uint64_t* key,
                                                const int* se) {
  const int lane = lane_id();
  int base = 0;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const uint64_t m = __ballot(vic[q]);
    if (vic[q]) {
      const int p = base + mbcnt(m);
      L.vkey[p] = key[q];
      L.vpack[p] = ((lane + WAVE * q) << 16) | (se[q] & 0xffff);
    }
    base += __popcll(m);
  }
}

template <int Q>
__device__ __forceinline__ int select_victims(LruLds& L, int S, int nins, const int* se,
                                              const long long* sst, const bool* ev) {
  const int lane = lane_id();
  int nev = 0;
  bool wide = false;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    nev += __popcll(__ballot(ev[q]));
    wide |= ev[q] && (sst[q] >> 32) != 0;
  }
  const int nact = nins < nev ? nins : nev;
  if (nact == 0) return 0;

  if (!__ballot(wide)) {
    // ---- every evictable stamp fits 32 bits -------------------------------------------------
    uint32_t mn = ~0u, mx = 0;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const uint32_t x = (uint32_t)sst[q];
      if (ev[q]) {
        mn = x < mn ? x : mn;
        mx = x > mx ? x : mx;
      }
    }
    wave_minmax_u32(mn, mx);
    uint64_t g[Q];
    int cnt0 = 0;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      g[q] = __ballot(ev[q] && (uint32_t)sst[q] == mn);
      cnt0 += __popcll(g[q]);
    }
    if (cnt0 >= nact) {
      // all victims from the oldest group, in slot order
      int base = 0;
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const int p = base + mbcnt(g[q]);
        if (((g[q] >> lane) & 1ull) && p < nact) put_victim(L, p, lane + WAVE * q, se[q]);
        base += __popcll(g[q]);
      }
      return nact;
    }
    // boundary stamp: tau = the nact-th smallest rel (#{rel < tau} < nact <= #{rel <= tau}),
    // found 8 bits at a time from the top of the range: each pass counts, in an LDS histogram,
    // the next digit of the slots whose higher digits equal tau's so far, and one wave scan
    // over the 256 bins finds the bin where the running count reaches nact
    uint32_t rel[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) rel[q] = ev[q] ? (uint32_t)sst[q] - mn : ~0u;
    const int b = 32 - __clz(mx - mn);              // mx > mn here: cnt0 < nact <= nev
    uint32_t tau = 0;
    int clt = 0;                                    // #{rel < tau's prefix so far}
    for (int sh = ((b - 1) >> 3) << 3; sh >= 0; sh -= 8) {
      *reinterpret_cast<int4*>(&L.hist[4 * lane]) = make_int4(0, 0, 0, 0);
      wave_lds_sync();
      const bool top = sh + 8 >= 32;
      const uint32_t pre = top ? 0u : tau >> (sh + 8);
#pragma unroll
      for (int q = 0; q < Q; ++q)
        if (ev[q] && (top || (rel[q] >> (sh + 8)) == pre))
          atomicAdd(&L.hist[(rel[q] >> sh) & 255u], 1);
      wave_lds_sync();
      const int4 h = *reinterpret_cast<const int4*>(&L.hist[4 * lane]);
      const int sum = h.x + h.y + h.z + h.w;
      const int c0 = clt + wave_incl_scan(sum) - sum;   // counted before this lane's bins
      const int c1 = c0 + h.x, c2 = c1 + h.y, c3 = c2 + h.z, c4 = c3 + h.w;
      int d = -1, cb = 0;
      if (c0 < nact && nact <= c1) {
        d = 0;
        cb = c0;
      } else if (c1 < nact && nact <= c2) {
        d = 1;
        cb = c1;
      } else if (c2 < nact && nact <= c3) {
        d = 2;
        cb = c2;
      } else if (c3 < nact && nact <= c4) {
        d = 3;
        cb = c3;
      }
      const int ln = __ffsll((unsigned long long)__ballot(d >= 0)) - 1;   // exactly one lane
      tau |= (uint32_t)(4 * ln + readlane(d, ln)) << sh;
      clt = readlane(cb, ln);
    }
    const int need = nact - clt;                    // >= 1 taken from the tau group
    bool vic[Q];
    uint64_t key[Q];
    int base = 0;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const uint64_t m = __ballot(rel[q] == tau);
      const int p = base + mbcnt(m);
      vic[q] = rel[q] < tau || (rel[q] == tau && p < need);
      key[q] = ((uint64_t)rel[q] << 10) | (uint64_t)(lane + WAVE * q);
      base += __popcll(m);
    }
    compact_victims<Q>(L, vic, key, se);
    rank_compacted(L, nact);
    return nact;
  }

  // ---- general: search the reference key (stamp << 20) | slot, biased to unsigned ----------
  const uint64_t bias = 0x8000000000000000ull;
  uint64_t rel[Q];
  uint64_t lo = ~0ull, hi = 0;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const uint64_t k = (((uint64_t)sst[q] << SLOT_BITS) | (uint64_t)(lane + WAVE * q)) ^ bias;
    rel[q] = ev[q] ? k : ~0ull;
    if (ev[q]) {
      lo = k < lo ? k : lo;
      hi = k > hi ? k : hi;
    }
  }
  lo = wave_reduce64(lo, OpMin64());
  hi = wave_reduce64(hi, OpMax64());
#pragma unroll
  for (int q = 0; q < Q; ++q)
    if (ev[q]) rel[q] -= lo;
  const uint64_t span = hi - lo;
  int b = span ? 64 - __clzll(span) : 0;
  uint64_t T = 0;
  for (; b > 0; --b) {
    const uint64_t c1 = T | (1ull << (b - 1));
    int n1 = 0;
#pragma unroll
    for (int q = 0; q < Q; ++q) n1 += __popcll(__ballot(rel[q] < c1));
    if (n1 < nact) T = c1;
  }
  bool vic[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) vic[q] = ev[q] && rel[q] <= T;
  compact_victims<Q>(L, vic, rel, se);
  rank_compacted(L, nact);
  return nact;
}

// Wave 0 after the routed set is known: pick the victims among the slots whose expert is not
// routed (the other waves refresh the hit stamps meanwhile).
template <int Q>
__device__ __forceinline__ int wave0_slots(LruLds& L, int S, int nins, bool ins_ok,
                                           const int (&se)[QS], const long long (&sst)[QS]) {
  const int lane = lane_id();
  uint64_t sb[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) sb[q] = L.sbusy[q];   // uniform reads, one round trip
  bool ev[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int i = lane + WAVE * q;
    ev[q] = i < S && !((sb[q] >> lane) & 1ull);
  }
  if (!ins_ok || nins == 0) return 0;
  return select_victims<Q>(L, S, nins, se, sst, ev);
}

__device__ __forceinline__ int wave0_dispatch(LruLds& L, int S, int nins, bool ins_ok,
                                              const int (&se)[QS], const long long (&sst)[QS]) {
  switch ((S + WAVE - 1) / WAVE) {
#define RLU_Q(n) \
  case n: return wave0_slots<n>(L, S, nins, ins_ok, se, sst);
    RLU_Q(1) RLU_Q(2) RLU_Q(3) RLU_Q(4) RLU_Q(5) RLU_Q(6) RLU_Q(7) RLU_Q(8)
    RLU_Q(9) RLU_Q(10) RLU_Q(11) RLU_Q(12) RLU_Q(13) RLU_Q(14) RLU_Q(15) RLU_Q(16)
#undef RLU_Q
    default: return 0;
  }
}

// block-size arithmetic: shifts when bs is a power of two (always, in practice: 16)
struct Blk {
  int bs, sh;
  __device__ Blk(int b) : bs(b), sh((b & (b - 1)) == 0 ? __builtin_ctz(b) : -1) {}
  __device__ __forceinline__ int pad(int c) const {
    return sh >= 0 ? ((c + bs - 1) >> sh) << sh : (c + bs - 1) / bs * bs;
  }
  __device__ __forceinline__ int blk(int x) const { return sh >= 0 ? x >> sh : x / bs; }
};

// Align output helpers, called with either the LDS stage or the global outputs so that
// each call site compiles to LDS or global stores (no generic pointers).
__device__ __forceinline__ void fill_align(int* __restrict__ oh, int* __restrict__ oc,
                                           int* __restrict__ eh, int* __restrict__ ec, int Lsz,
                                           int NB, int mk, bool vec) {
  int k0 = 0;
  if (vec) {                                        // 16-byte stores (outputs 16-byte aligned)
    const int4 m4 = make_int4(mk, mk, mk, mk);
    for (int k = 4 * threadIdx.x; k + 4 <= Lsz; k += 4 * NT) {
      *reinterpret_cast<int4*>(oh + k) = m4;
      *reinterpret_cast<int4*>(oc + k) = m4;
    }
    k0 = Lsz & ~3;
  }
  for (int k = k0 + threadIdx.x; k < Lsz; k += NT) {
    oh[k] = mk;
    oc[k] = mk;
  }
  for (int k = threadIdx.x; k < NB; k += NT) {
    eh[k] = -1;
    ec[k] = -1;
  }
}

// The starts (cum_h / cum_c) and expert ids of a thread's buckets; with pad >= 0 also the
// padding entries of each bucket, [start + count, start + padded count), set to pad.
__device__ __forceinline__ void place_buckets(LruLds& L, int* __restrict__ oh,
                                              int* __restrict__ oc, int* __restrict__ eh,
                                              int* __restrict__ ec, const int (&ph)[EJ],
                                              const int (&pc)[EJ], int h0, int h1, int c0,
                                              int c1, int runa, int runb, int NB, const Blk& B,
                                              int pad) {
#pragma unroll
  for (int side = 0; side < 2; ++side) {
    const bool hs = side == 0;
    int run = hs ? runa : runb;
    const int i0 = hs ? h0 : c0, i1 = hs ? h1 : c1;
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
      const int c = hs ? ph[j] : pc[j];
      const int i = i0 + j;
      if (i < i1) {
        if (hs)
          L.cum_h[i] = run;
        else
          L.cum_c[i] = run;
        if (c > 0) {
          int* eo = hs ? eh : ec;
          for (int k = B.blk(run); k < B.blk(run + B.pad(c)); ++k)
            if (k < NB) eo[k] = i;
          if (pad >= 0) {
            int* so = hs ? oh : oc;
            for (int k = run + c; k < run + B.pad(c); ++k) so[k] = pad;
          }
        }
        run += B.pad(c);
      }
    }
  }
}

// tokens routed to expert e this step: its token bitmap (staged) or the atomic counts
__device__ __forceinline__ int expert_tokens(const LruLds& L, int e, bool staged) {
  if (!staged) return L.ecnt[e];
  int c = 0;
#pragma unroll
  for (int x = 0; x < TW; ++x) c += __popcll(L.tk.tmask[e][x]);
  return c;
}

// both align outputs start on a 16-byte boundary (the copy-out then stores 16-byte units)
static inline bool aligned16(const int* a, const int* b) {
  return (((uintptr_t)a | (uintptr_t)b) & 15) == 0;
}

// The post-update bucket of routed expert e: its slot when resident on entry or inserted now
// (the rank-mr miss takes victim slot vslot[mr]), else -1 (the cold list).
__device__ __forceinline__ int post_slot(const LruLds& L, int e, int S, int nact) {
  int s = L.tab[e];
  if ((unsigned)s < (unsigned)S) return s;
  if (nact > 0) {
    const uint64_t mw = L.rbits[e >> 6] & L.nres[e >> 6];
    if ((mw >> (e & 63)) & 1ull) {
      const int mr = L.mpre[e >> 6] + __popcll(mw & ((1ull << (e & 63)) - 1ull));
      if (mr < nact) return L.vslot[mr];
    }
  }
  return -1;
}

// The step's install count as any wave can derive it from the routed, non-resident and
// busy-slot bitmaps -- the number wave 0's victim search arrives at: nins = the misses (in
// ascending expert id) up to max_inserts, none on a read-through step (more than max_distinct
// experts routed); nact = min(nins, evictable slots). Also writes this wave's copy of the
// per-bitmap-word miss prefix (mp[w] = misses in words below w).
struct InsCount {
  int nins, nact;
};
__device__ __forceinline__ InsCount insert_counts(const LruLds& L, int S, int max_distinct,
                                                  int max_inserts, int* mp) {
  const int lane = lane_id();
  uint64_t rw = 0, nw = 0, sb = 0;
  if (lane < NWORD) {
    rw = L.rbits[lane];
    nw = L.nres[lane];
    sb = L.sbusy[lane];
  }
  const int distinct = readlane(row_sum(__popcll(rw)), 0);          // words live in row 0
  const int busy = readlane(row_sum(__popcll(sb)), 0);
  const int mpop = __popcll(rw & nw);
  const int mincl = row_incl_scan(mpop);
  const int total = readlane(mincl, NWORD - 1);
  if (lane < NWORD) mp[lane] = mincl - mpop;
  InsCount r;
  r.nins = distinct <= max_distinct ? (total < max_inserts ? total : max_inserts) : 0;
  const int nev = S - busy;
  r.nact = r.nins < nev ? r.nins : nev;
  return r;
}

// The per-token-group-128 quant of the layer's hidden state, run by workgroups 1.. of the fused
// launch while workgroup 0 runs the cache: the two are independent and both feed the first
// GEMM, so one launch serves both. One row per wave: the launch's LDS footprint leaves room for
// one workgroup per CU, so a prefill chunk's rows go four to a workgroup.
struct QuantJob {
  const uint16_t* x;
  int rows, K, ldx;
  uint8_t* q;
  float* scale;
};

// BSC: the align block size as a compile-time constant (16, the size every decode call uses),
// or 0 to take bs at run time
template <bool ALIGN, int BSC = 0>
__global__ __launch_bounds__(NT) void lru_k(
    const int* __restrict__ ids, int mk, int E, int S, int max_distinct, int max_inserts,
    int* __restrict__ table, int* __restrict__ map_cold, int* __restrict__ slot_expert,
    long long* __restrict__ slot_stamp, unsigned char* __restrict__ routed,
    long long* __restrict__ step, int* __restrict__ miss, int* __restrict__ n_miss, int bs,
    int Lsz, int NB, int* __restrict__ sorted_hot, int* __restrict__ eids_hot,
    int* __restrict__ npad_hot, int* __restrict__ sorted_cold, int* __restrict__ eids_cold,
    int* __restrict__ npad_cold, QuantJob qj, bool vec_out, bool defer_place) {
  if (blockIdx.x > 0) {                          // quant workgroups: one row per wave
    const int r = (blockIdx.x - 1) * NW + (int)threadIdx.x / WAVE;
    if (r < qj.rows)
      wave_quant_row128(qj.x + (size_t)r * qj.ldx, qj.K, qj.q + (size_t)r * qj.K,
                        qj.scale + (size_t)r * (qj.K / 128));
    return;
  }
  __shared__ LruLds L;
  const int t = threadIdx.x;
  const int w = t / WAVE;
  const int lane = lane_id();
  // Decode-sized calls stage both align outputs in LDS, so every output element is written
  // to global memory exactly once, by coalesced stores at the end. Larger ones pre-fill the
  // outputs in global memory and overwrite them after a full barrier.
  const bool staged = ALIGN && mk <= NT && Lsz <= LSTAGE && NB <= NBSTAGE;

  // ---- loads, all issued before any barrier --------------------------------------------
  const long long st = step[0] + 1;
  int tab[EJ];
#pragma unroll
  for (int j = 0; j < EJ; ++j) {
    const int e = t + NT * j;
    tab[j] = e < E ? table[e] : 0;
  }
  int se[QS];
  long long sst[QS];
  if (w == 0) {
#pragma unroll
    for (int q = 0; q < QS; ++q) {
      const int i = lane + WAVE * q;
      se[q] = i < S ? slot_expert[i] : -1;
      sst[q] = i < S ? slot_stamp[i] : 0;
    }
  }
  const int tok0 = t < mk ? ids[t] : -1;
  const bool v0 = tok0 >= 0 && tok0 < E;

  // ---- init -------------------------------------------------------------------------------
  if (ALIGN) {
    if (staged) {
      if (v0) {                                  // clear the masks this step will use
#pragma unroll
        for (int x = 0; x < TW; ++x) L.tk.tmask[tok0][x] = 0;
      }
    } else {
      reinterpret_cast<uint4*>(&L.tk.wcnt[0][0])[t] = make_uint4(0, 0, 0, 0);
      // deferred placement: place_k writes all of the sorted arrays, sentinels included
      fill_align(sorted_hot, sorted_cold, eids_hot, eids_cold, defer_place ? 0 : Lsz, NB, mk,
                 vec_out);
    }
    for (int i = t; i < S; i += NT) {
      L.cnt_h[i] = 0;
      L.vrank[i] = -1;
    }
  }
#pragma unroll
  for (int j = 0; j < EJ; ++j) {
    const int e = t + NT * j;
    const uint64_t nr = __ballot(e < E && tab[j] < 0);
    if (lane == 0) L.nres[j * NW + w] = nr;
    if (e < E) {
      L.tab[e] = tab[j];
      L.ecnt[e] = 0;
    }
  }
  if (t < NWORD) {
    L.rbits[t] = 0;
    L.sbusy[t] = 0;
  }
  if (ALIGN && !staged)
    __syncthreads();  // 1 -- full: the global sentinel stores complete before any overwrite
  else
    lds_barrier();    // 1

  // ---- mark routed experts and their slots; per-expert token sets. The general align path
  // only counts tokens per expert here (one atomic per token): its routed and busy-slot
  // bitmaps follow from the counts after the barrier --------------------------------------
  const bool count_only = ALIGN && !staged;
  auto mark = [&](int e, int i) {
    if (count_only) {
      if (e >= 0 && e < E) atomicAdd(&L.ecnt[e], 1);
    } else if (e >= 0 && e < E) {
      atomicOr(reinterpret_cast<unsigned long long*>(&L.rbits[e >> 6]), 1ull << (e & 63));
      const int s = L.tab[e];
      if ((unsigned)s < (unsigned)S)
        atomicOr(reinterpret_cast<unsigned long long*>(&L.sbusy[s >> 6]), 1ull << (s & 63));
      if (ALIGN) {
        if (staged)
          atomicOr(reinterpret_cast<unsigned long long*>(&L.tk.tmask[e][i >> 6]),
                   1ull << (i & 63));
        else
          atomicAdd(&L.ecnt[e], 1);
      }
    }
  };
  if (t < mk) mark(tok0, t);
  int mark_from = NT;
  if (count_only && (((uintptr_t)ids & 15) == 0) && mk > NT) {
    mark_from = NT + ((mk - NT) & ~3);
    count_ids_vec(ids, NT, mark_from, E, L.ecnt);
    if (t < mk - mark_from) mark(ids[mark_from + t], mark_from + t);
    mark_from = mk;
  }
  for (int i = t + mark_from; i < mk; i += MLOADS * NT) {  // MLOADS loads in flight
    int e[MLOADS];
#pragma unroll
    for (int u = 0; u < MLOADS; ++u) e[u] = ids[min(i + u * NT, mk - 1)];
#pragma unroll
    for (int u = 0; u < MLOADS; ++u)
      if (i + u * NT < mk) mark(e[u], i + u * NT);
  }
  const int kbits = E > 1 ? 32 - __clz(E - 1) : 0;
  int inrank = 0;
  if (ALIGN && !staged) {
    const uint64_t m = match_any(tok0, v0, kbits);
    inrank = mbcnt(m);
    if (v0 && inrank == 0) L.tk.wcnt[w][tok0] = (uint8_t)__popcll(m);
  }
  lds_barrier();  // 2
  if (count_only) {
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
      const int e = t + NT * j;
      const bool r = e < E && L.ecnt[e] > 0;
      const uint64_t rw = __ballot(r);
      if (lane == 0) L.rbits[j * NW + w] = rw;
      if (r && (unsigned)tab[j] < (unsigned)S)
        atomicOr(reinterpret_cast<unsigned long long*>(&L.sbusy[tab[j] >> 6]),
                 1ull << (tab[j] & 63));
    }
    lds_barrier();  // 2b
  }

  // ---- wave 0: distinct count, miss ranks, victims; the other waves meanwhile do what does
  // not depend on the victims: hit stamps, routed flags, bucket counts of every expert that
  // is not a miss --------------------------------------------------------------------------
  if (w == 0) {
    uint64_t rw = 0, nw = 0;
    if (lane < NWORD) {
      rw = L.rbits[lane];
      nw = L.nres[lane];
    }
    const int distinct = readlane(row_sum(__popcll(rw)), 0);          // words live in row 0
    const int mpop = __popcll(rw & nw);
    const int mincl = row_incl_scan(mpop);
    const int total = readlane(mincl, NWORD - 1);
    if (lane < NWORD) L.mpre[lane] = mincl - mpop;
    const bool ins_ok = distinct <= max_distinct;
    const int nins = ins_ok ? (total < max_inserts ? total : max_inserts) : 0;
    const int nact = wave0_dispatch(L, S, nins, ins_ok, se, sst);
    if (lane == 0) {
      L.misc[0] = nact;
      L.misc[1] = nins;
    }
  } else {
    const uint64_t rw = lane < NWORD ? L.rbits[lane] : 0ull;
    const bool ins_ok = readlane(row_sum(__popcll(rw)), 0) <= max_distinct;
    // with the align, the misses' buckets too: how many misses get a slot follows from the
    // bitmaps alone (wave 0's search only decides which slots), so a miss of rank < nact
    // leaves its token count for the slot it takes (vcnt) and the others go cold
    const InsCount ic = ALIGN ? insert_counts(L, S, max_distinct, max_inserts, L.mpw[w])
                              : InsCount{0, 0};
    if (ALIGN) wave_lds_sync();
    if (ins_ok) {                                    // hit: r4d_lru.hip:228-238
      for (int i = t - WAVE; i < S; i += NT - WAVE)
        if (bit_of(L.sbusy, i)) slot_stamp[i] = st;
    }
    for (int e = t - WAVE; e < E; e += NT - WAVE) {
      const bool r = bit_of(L.rbits, e);
      routed[e] = r ? 1 : 0;
      const int s0 = L.tab[e];
      if (ALIGN) {
        const int c = r ? expert_tokens(L, e, staged) : 0;
        if (r && s0 < 0) {
          const uint64_t mw = L.rbits[e >> 6] & L.nres[e >> 6];
          const int rank = L.mpw[w][e >> 6] + __popcll(mw & ((1ull << (e & 63)) - 1ull));
          if (rank < ic.nins) L.vexp[rank] = e;
          if (rank < ic.nact) L.vcnt[rank] = c;
          L.cnt_c[e] = rank < ic.nact ? 0 : c;
        } else {
          const bool hot = r && (unsigned)s0 < (unsigned)S;
          if (hot) L.cnt_h[s0] = c;
          L.cnt_c[e] = (r && !hot) ? c : 0;
        }
        L.ecnt[e] = 0;  // general path: becomes the running per-expert base of the chunks
      }
    }
  }
  lds_barrier();  // 3

  const int nact = L.misc[0];
  const int nins = L.misc[1];

  // ---- misses: miss list and installs (global stores only: every bucket count is in LDS
  // already, so the scans below start without another barrier). With the align the misses come
  // by rank from vexp (one thread per rank); without it each thread checks its experts ------
  auto install = [&](int rank, int e) __attribute__((always_inline)) {
    if (rank < nins) miss[2 * rank] = e;
    if (rank < nact) {
      const int sl = L.vslot[rank];
      const int old = L.vold[rank];
      if (old >= 0 && old < E) {
        table[old] = -1;
        map_cold[old] = old;
      }
      table[e] = sl;
      map_cold[e] = -1;
      slot_expert[sl] = e;
      slot_stamp[sl] = st;
      miss[2 * rank + 1] = sl;
    }
  };
  if (ALIGN) {
    for (int r = t; r < nins; r += NT) install(r, L.vexp[r]);
  } else {
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
      const int e = t + NT * j;
      if (e >= E) continue;
      if (!(tab[j] < 0 && bit_of(L.rbits, e)) || nins == 0) continue;
      const uint64_t mw = L.rbits[e >> 6] & L.nres[e >> 6];
      install(L.mpre[e >> 6] + __popcll(mw & ((1ull << (e & 63)) - 1ull)), e);
    }
  }
  if (t == 0) {
    step[0] = st;
    n_miss[0] = nact;
  }
  if (!ALIGN) return;

  // ---- block-padded exclusive scans: thread t owns a contiguous run of slots and experts ---
  const Blk B(BSC ? BSC : bs);
  const int Ch = (S + NT - 1) / NT, Ce = (E + NT - 1) / NT;
  const int h0 = t * Ch, h1 = min(h0 + Ch, S);
  const int c0 = t * Ce, c1 = min(c0 + Ce, E);
  int ph[EJ], pc[EJ], a = 0, b = 0;
#pragma unroll
  for (int j = 0; j < EJ; ++j) {
    // a slot's bucket: its resident expert's tokens, or those of the miss installed in it
    int hv = 0;
    if (j < Ch && h0 + j < h1) {
      const int vr = L.vrank[h0 + j];
      hv = L.cnt_h[h0 + j] + (vr >= 0 ? L.vcnt[vr] : 0);
    }
    ph[j] = hv;
    pc[j] = (j < Ce && c0 + j < c1) ? L.cnt_c[c0 + j] : 0;
    a += B.pad(ph[j]);
    b += B.pad(pc[j]);
  }
  const int ai = wave_incl_scan(a), bi = wave_incl_scan(b);
  if (lane == WAVE - 1) {
    L.wsum[w][0] = ai;
    L.wsum[w][1] = bi;
  }
  lds_barrier();  // 4
  int runa = ai - a, runb = bi - b, tota = 0, totb = 0;
#pragma unroll
  for (int x = 0; x < NW; ++x) {
    const int ya = L.wsum[x][0], yb = L.wsum[x][1];
    if (x < w) {
      runa += ya;
      runb += yb;
    }
    tota += ya;
    totb += yb;
  }
  if (t == 0) {
    npad_hot[0] = tota;
    npad_cold[0] = totb;
  }
  // bucket starts and expert ids; staged: every entry below num_post_pad starts as the
  // sentinel (the tokens overwrite theirs after the barrier)
  if (staged) {
    const int4 m4 = make_int4(mk, mk, mk, mk);
    for (int k = 4 * t; k < tota; k += 4 * NT) *reinterpret_cast<int4*>(&L.stage_h[k]) = m4;
    for (int k = 4 * t; k < totb; k += 4 * NT) *reinterpret_cast<int4*>(&L.stage_c[k]) = m4;
    place_buckets(L, L.stage_h, L.stage_c, L.stage_eh, L.stage_ec, ph, pc, h0, h1, c0, c1, runa,
                  runb, NB, B, -1);
  } else
    place_buckets(L, sorted_hot, sorted_cold, eids_hot, eids_cold, ph, pc, h0, h1, c0, c1, runa,
                  runb, NB, B, -1);
  lds_barrier();  // 5

  if (staged) {
    // ---- each token places itself: its bucket's start plus the number of the bucket's tokens
    // with a smaller index (the set bits of its expert's token mask below it), so every bucket
    // lists its tokens in index order --------------------------------------------------------
    if (v0) {
      const int e = tok0;
      int rank = __popcll(L.tk.tmask[e][t >> 6] & ((1ull << (t & 63)) - 1ull));
#pragma unroll
      for (int wd = 0; wd < TW; ++wd)
        if (wd < (t >> 6)) rank += __popcll(L.tk.tmask[e][wd]);
      const int s = post_slot(L, e, S, nact);
      const int pos = (s >= 0 ? L.cum_h[s] : L.cum_c[e]) + rank;
      if (pos < Lsz) {
        if (s >= 0)
          L.stage_h[pos] = t;
        else
          L.stage_c[pos] = t;
      }
    }
    lds_barrier();  // 6
    // ---- copy the staged outputs out, coalesced; past num_post_pad the sentinels ------------
    const int nbh = B.blk(tota), nbc = B.blk(totb);
    int k0 = 0;
    if (vec_out) {                                  // 16-byte stores (outputs 16-byte aligned)
      for (int k = 4 * t; k + 4 <= Lsz; k += 4 * NT) {
        // LDS read first, then a value select (a select of the source would become a generic
        // load from LDS or from a private copy of the sentinel)
        const int4 h = *reinterpret_cast<const int4*>(&L.stage_h[k]);
        const int4 c = *reinterpret_cast<const int4*>(&L.stage_c[k]);
        const bool ih = k < tota, ic = k < totb;
        *reinterpret_cast<int4*>(sorted_hot + k) =
            make_int4(ih ? h.x : mk, ih ? h.y : mk, ih ? h.z : mk, ih ? h.w : mk);
        *reinterpret_cast<int4*>(sorted_cold + k) =
            make_int4(ic ? c.x : mk, ic ? c.y : mk, ic ? c.z : mk, ic ? c.w : mk);
      }
      k0 = Lsz & ~3;
    }
    for (int k = k0 + t; k < Lsz; k += NT) {
      sorted_hot[k] = k < tota ? L.stage_h[k] : mk;
      sorted_cold[k] = k < totb ? L.stage_c[k] : mk;
    }
    for (int k = t; k < NB; k += NT) {
      eids_hot[k] = k < nbh ? L.stage_eh[k] : -1;
      eids_cold[k] = k < nbc ? L.stage_ec[k] : -1;
    }
    return;
  }

  if (defer_place) return;                        // place_k ranks the tokens in parallel

  // ---- general placement, chunk by chunk of NT tokens in index order ---------------------
  // the next chunk's id is loaded one chunk ahead, so no chunk waits for a memory round trip
  int nxt = NT + t < mk ? ids[NT + t] : -1;
  for (int c = 0; c * NT < mk; ++c) {
    const int i = c * NT + t;
    int e = tok0;
    bool v = v0;
    if (c > 0) {
      const int cur = nxt;
      const int in = (c + 1) * NT + t;
      nxt = in < mk ? ids[in] : -1;
      lds_barrier();
      // fold the previous chunk's per-wave counts into the per-expert base, then rank this one
#pragma unroll
      for (int j = 0; j < EJ; ++j) {
        const int x = t + NT * j;
        if (x < E) {
          int add = 0;
#pragma unroll
          for (int ww = 0; ww < NW; ++ww) {
            add += L.tk.wcnt[ww][x];
            L.tk.wcnt[ww][x] = 0;
          }
          L.ecnt[x] += add;
        }
      }
      e = i < mk ? cur : -1;
      v = e >= 0 && e < E;
      lds_barrier();
      const uint64_t m = match_any(e, v, kbits);
      inrank = mbcnt(m);
      if (v && inrank == 0) L.tk.wcnt[w][e] = (uint8_t)__popcll(m);
      lds_barrier();
    }
    if (v) {
      int rank = L.ecnt[e] + inrank;
      for (int ww = 0; ww < w; ++ww) rank += L.tk.wcnt[ww][e];
      const int s = post_slot(L, e, S, nact);
      if (s >= 0) {
        const int pos = L.cum_h[s] + rank;
        if (pos < Lsz) sorted_hot[pos] = i;
      } else {
        const int pos = L.cum_c[e] + rank;
        if (pos < Lsz) sorted_cold[pos] = i;
      }
    }
  }
}

// grid = (chunks, lanes), block = 256: block (c, j) copies misses j, j + lanes, ... ; within
// a slab, 16-byte vectors are spread over the `chunks` blocks, four loads in flight per lane.
// Destinations are written non-temporally: a gathered slab is read by the next GEMM once.
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(NT) void gather_k(v4u* d0, const v4u* s0, long v0,
                                               v4u* d1, const v4u* s1, long v1,
                                               v4u* d2, const v4u* s2, long v2,
                                               v4u* d3, const v4u* s3, long v3,
                                               v4u* d4, const v4u* s4, long v4,
                                               v4u* d5, const v4u* s5, long v5,
                                               const int* __restrict__ miss,
                                               const int* __restrict__ n_miss) {
  const int nm = n_miss[0];
  const long stride = (long)gridDim.x * NT;
  const long start = (long)blockIdx.x * NT + threadIdx.x;
  for (int j = blockIdx.y; j < nm; j += gridDim.y) {
    const long e = miss[2 * j], sl = miss[2 * j + 1];
    v4u* dd[6] = {d0, d1, d2, d3, d4, d5};
    const v4u* ss[6] = {s0, s1, s2, s3, s4, s5};
    const long vv[6] = {v0, v1, v2, v3, v4, v5};
#pragma unroll
    for (int b = 0; b < 6; ++b) {
      const v4u* __restrict__ p = ss[b] + e * vv[b];
      v4u* __restrict__ q = dd[b] + sl * vv[b];
      const long V = vv[b];
      long i = start;
      for (; i + 3 * stride < V; i += 4 * stride) {
        const v4u x0 = p[i], x1 = p[i + stride], x2 = p[i + 2 * stride], x3 = p[i + 3 * stride];
        __builtin_nontemporal_store(x0, q + i);
        __builtin_nontemporal_store(x1, q + i + stride);
        __builtin_nontemporal_store(x2, q + i + 2 * stride);
        __builtin_nontemporal_store(x3, q + i + 3 * stride);
      }
      for (; i < V; i += stride) __builtin_nontemporal_store(p[i], q + i);
    }
  }
}

// Splits the hot align's block expert ids (slot indices) by whether this step's gather
// writes the slot: eids_res keeps the slots resident before the manager ran (-1 elsewhere),
// eids_new keeps the slots the manager just installed (the miss list's slot column). A GEMM
// over eids_res needs no gathered byte, so it can run while the gather copies; one over
// eids_new runs after it. Every block lands in exactly one of the two (or neither, for -1).
// One workgroup: a slot bitmap in LDS, then one pass over the blocks.
__global__ __launch_bounds__(NT) void split_fresh_k(const int* __restrict__ eids, int nb,
                                                    const int* __restrict__ miss,
                                                    const int* __restrict__ n_miss, int cap,
                                                    int S, int* __restrict__ eids_res,
                                                    int* __restrict__ eids_new) {
  __shared__ unsigned char fresh[MAXS];
  for (int s = threadIdx.x; s < S; s += NT) fresh[s] = 0;
  __syncthreads();
  const int nm = min(n_miss[0], cap);
  for (int j = threadIdx.x; j < nm; j += NT) {
    const int sl = miss[2 * j + 1];
    if ((unsigned)sl < (unsigned)S) fresh[sl] = 1;
  }
  __syncthreads();
  for (int b = threadIdx.x; b < nb; b += NT) {
    const int s = eids[b];
    const bool f = (unsigned)s < (unsigned)S && fresh[s];
    eids_res[b] = f ? -1 : s;
    eids_new[b] = f ? s : -1;
  }
}

// ---- placement for large token counts, many workgroups ----------------------------------
// Above PLACE_MIN tokens the fused launch stops once the expert-id sentinels, the bucket
// counts, starts, expert ids and num_post_pad are written; place_k writes everything of the
// sorted arrays. Workgroup c (PT threads) takes tokens [c PT, (c + 1) PT):
//  * it counts every id per expert, and separately those before its own tokens (LDS atomics;
//    order does not matter for a count);
//  * it ranks its own tokens in index order (bit-sliced wave match + per-wave counts), as the
//    single-workgroup loop does, so every bucket lists its tokens in ascending index order;
//  * it writes the padding sentinels of its share of the experts' buckets, [start + count,
//    start + padded count), and its share of [num_post_pad, L).
// Token positions, padding and the tail are disjoint, so no two workgroups write one entry.
// A routed expert's bucket is its slot in the updated table (hot) or itself (cold); a bucket
// starts at the first block of its run in eids_hot / eids_cold. The host takes this route only
// when NB * bs >= L: then every bucket that starts below L has its first block recorded, and
// the others (start left at L) write nothing.
constexpr int PT = 1024;            // threads and tokens of one placement workgroup
constexpr int PWV = PT / WAVE;
constexpr int PLACE_MIN = 1536;     // the fused launch defers placement above this many tokens
constexpr int PLOADS = 8;           // id loads in flight per thread while counting (unaligned)
constexpr int PB = 4;               // expert-id blocks per thread in flight

struct PlaceLds {
  int start_h[MAXS];
  int start_c[MAXE];
  int before[MAXE];                 // tokens of the expert before this workgroup's
  int total[MAXE];                  // tokens of the expert in the step
  int tab[MAXE];                    // updated table
  alignas(16) uint8_t wcnt[PWV][MAXE];  // tokens of the expert per wave among this chunk
};

__device__ __forceinline__ void count2(PlaceLds& P, int e, int i, int c0, int E) {
  if ((unsigned)e < (unsigned)E) {
    atomicAdd(&P.total[e], 1);
    if (i < c0) atomicAdd(&P.before[e], 1);
  }
}

__global__ __launch_bounds__(PT) void place_k(const int* __restrict__ ids, int mk, int E, int S,
                                              const int* __restrict__ table,
                                              const int* __restrict__ eids_hot,
                                              const int* __restrict__ eids_cold,
                                              const int* __restrict__ npad_hot,
                                              const int* __restrict__ npad_cold, int NB, int bs,
                                              int Lsz, int* __restrict__ sorted_hot,
                                              int* __restrict__ sorted_cold) {
  __shared__ PlaceLds P;
  const int t = threadIdx.x, w = t / WAVE;
  const int c0 = blockIdx.x * PT, c1 = min(c0 + PT, mk);
  // this workgroup's id and the table first: nothing below waits on a load it does not need
  const int own = ids[min(c0 + t, c1 - 1)];
  const int tb = table[min(t, E - 1)];              // E <= MAXE == PT
  const int nph = npad_hot[0], npc = npad_cold[0];
  if (t < S) P.start_h[t] = Lsz;
  if (t < E) {
    P.start_c[t] = Lsz;
    P.before[t] = 0;
    P.total[t] = 0;
    P.tab[t] = tb;
  }
  reinterpret_cast<uint4*>(&P.wcnt[0][0])[t] = make_uint4(0, 0, 0, 0);   // PWV * MAXE bytes
  lds_barrier();
  // the first block of each bucket's run; PB blocks per thread in flight
  for (int b0 = 0; b0 < NB; b0 += PB * PT) {
    int eh[PB], ec[PB], ph[PB], pc[PB];
#pragma unroll
    for (int u = 0; u < PB; ++u) {
      const int b = min(b0 + t + u * PT, NB - 1), bp = max(b - 1, 0);
      eh[u] = eids_hot[b];
      ec[u] = eids_cold[b];
      ph[u] = eids_hot[bp];
      pc[u] = eids_cold[bp];
    }
#pragma unroll
    for (int u = 0; u < PB; ++u) {
      const int b = b0 + t + u * PT;
      if (b < NB) {
        if ((unsigned)eh[u] < (unsigned)S && (b == 0 || eh[u] != ph[u])) P.start_h[eh[u]] = b * bs;
        if ((unsigned)ec[u] < (unsigned)E && (b == 0 || ec[u] != pc[u])) P.start_c[ec[u]] = b * bs;
      }
    }
  }
  // every id, per expert: VL 16-byte loads in flight per thread when ids is 16-byte aligned
  if ((((uintptr_t)ids & 15) == 0)) {
    const int4* v = reinterpret_cast<const int4*>(ids);
    const int nv = mk / 4;
    for (int j = t; j < nv; j += VL * PT) {
      int4 x[VL];
#pragma unroll
      for (int u = 0; u < VL; ++u) x[u] = v[min(j + u * PT, nv - 1)];
#pragma unroll
      for (int u = 0; u < VL; ++u) {
        const int q = j + u * PT;
        if (q < nv) {
          count2(P, x[u].x, 4 * q, c0, E);
          count2(P, x[u].y, 4 * q + 1, c0, E);
          count2(P, x[u].z, 4 * q + 2, c0, E);
          count2(P, x[u].w, 4 * q + 3, c0, E);
        }
      }
    }
    if (t < mk - 4 * nv) count2(P, ids[4 * nv + t], 4 * nv + t, c0, E);
  } else {
    for (int i = t; i < mk; i += PLOADS * PT) {
      int x[PLOADS];
#pragma unroll
      for (int u = 0; u < PLOADS; ++u) x[u] = ids[min(i + u * PT, mk - 1)];
#pragma unroll
      for (int u = 0; u < PLOADS; ++u)
        if (i + u * PT < mk) count2(P, x[u], i + u * PT, c0, E);
    }
  }
  lds_barrier();
  // this workgroup's tokens, in index order
  const int kbits = E > 1 ? 32 - __clz(E - 1) : 0;
  const int i = c0 + t;
  const int e = i < c1 ? own : -1;
  const bool v = (unsigned)e < (unsigned)E;
  const uint64_t m = match_any(e, v, kbits);
  const int inrank = mbcnt(m);
  if (v && inrank == 0) P.wcnt[w][e] = (uint8_t)__popcll(m);
  lds_barrier();
  if (v) {
    int rank = P.before[e] + inrank;
    for (int ww = 0; ww < w; ++ww) rank += P.wcnt[ww][e];
    const int sl = P.tab[e];
    const bool hot = (unsigned)sl < (unsigned)S;
    const int pos = (hot ? P.start_h[sl] : P.start_c[e]) + rank;
    if (pos < Lsz) {
      if (hot)
        sorted_hot[pos] = i;
      else
        sorted_cold[pos] = i;
    }
  }
  // padding of this workgroup's experts (one per thread), then its share of the tails
  const int ex = blockIdx.x + gridDim.x * t;
  if (ex < E) {
    const int cnt = P.total[ex];
    if (cnt > 0) {
      const int sl = P.tab[ex];
      const bool hot = (unsigned)sl < (unsigned)S;
      const int st = hot ? P.start_h[sl] : P.start_c[ex];
      const int end = min(st + (cnt + bs - 1) / bs * bs, Lsz);
      for (int p = st + cnt; p < end; ++p) {
        if (hot)
          sorted_hot[p] = mk;
        else
          sorted_cold[p] = mk;
      }
    }
  }
  for (int p = max(nph, 0) + blockIdx.x * PT + t; p < Lsz; p += gridDim.x * PT) sorted_hot[p] = mk;
  for (int p = max(npc, 0) + blockIdx.x * PT + t; p < Lsz; p += gridDim.x * PT) sorted_cold[p] = mk;
}

// Placement moves to place_k for large token counts when every bucket start below L is
// recorded in the block ids (NB blocks of bs cover L).
static inline bool defer_placement(int mk, int bs, int L, int NB) {
  return mk > PLACE_MIN && (long long)NB * bs >= L;
}

static inline void launch_place(const int* ids, int mk, int E, int S, const int* table,
                                const int* eids_hot, const int* eids_cold, const int* npad_hot,
                                const int* npad_cold, int NB, int bs, int L, int* sorted_hot,
                                int* sorted_cold, hipStream_t stream) {
  hipLaunchKernelGGL(place_k, dim3((mk + PT - 1) / PT), dim3(PT), 0, stream, ids, mk, E, S,
                     table, eids_hot, eids_cold, npad_hot, npad_cold, NB, bs, L, sorted_hot,
                     sorted_cold);
}

}  // namespace rlu

extern "C" {

// kernels/lru/r4d_lru.hip:579-589
int r4d_lru_manage(const int* topk_ids, int mk, int E, int S, int max_distinct,
                   int max_inserts, int* table, int* map_cold, int* slot_expert,
                   long long* slot_stamp, unsigned char* routed, long long* step, int* miss,
                   int* n_miss, hipStream_t stream) {
  if (E <= 0 || E > rlu::MAXE || S <= 0 || S > rlu::MAXS) return -1;
  if (max_inserts < 0 || max_inserts > rlu::MAXINS) return -1;
  if (mk < 0) mk = 0;     // the reference's loops over mk ids run zero times
  hipLaunchKernelGGL(rlu::lru_k<false>, dim3(1), dim3(rlu::NT), 0, stream, topk_ids, mk, E, S,
                     max_distinct, max_inserts, table, map_cold, slot_expert, slot_stamp,
                     routed, step, miss, n_miss, 1, 0, 0, nullptr, nullptr, nullptr, nullptr,
                     nullptr, nullptr, rlu::QuantJob{}, false, false);
  return (int)hipGetLastError();
}

// kernels/lru/r4d_lru.hip:596-610
int r4d_lru_fused(const int* topk_ids, int mk, int E, int S, int max_distinct,
                  int max_inserts, int* table, int* map_cold, int* slot_expert,
                  long long* slot_stamp, unsigned char* routed, long long* step, int* miss,
                  int* n_miss, int bs, int L, int NB, int* sorted_hot, int* eids_hot,
                  int* npad_hot, int* sorted_cold, int* eids_cold, int* npad_cold,
                  hipStream_t stream) {
  if (E <= 0 || E > rlu::MAXE || S <= 0 || S > rlu::MAXS) return -1;
  if (bs <= 0 || L <= 0 || NB <= 0 || mk < 0) return -1;
  if (max_inserts < 0 || max_inserts > rlu::MAXINS) return -1;
  const bool defer = rlu::defer_placement(mk, bs, L, NB);
  auto k = bs == 16 ? rlu::lru_k<true, 16> : rlu::lru_k<true, 0>;
  hipLaunchKernelGGL(k, dim3(1), dim3(rlu::NT), 0, stream, topk_ids, mk, E, S, max_distinct,
                     max_inserts, table, map_cold, slot_expert, slot_stamp, routed, step, miss,
                     n_miss, bs, L, NB, sorted_hot, eids_hot, npad_hot, sorted_cold, eids_cold,
                     npad_cold, rlu::QuantJob{}, rlu::aligned16(sorted_hot, sorted_cold), defer);
  if (defer)
    rlu::launch_place(topk_ids, mk, E, S, table, eids_hot, eids_cold, npad_hot, npad_cold, NB,
                      bs, L, sorted_hot, sorted_cold, stream);
  return (int)hipGetLastError();
}

// r4d_lru_fused plus, in the same launch, the per-token-group-128 e4m3 quant of x [rows, K]
// bf16 (ldx elements apart) into q [rows, K] and scale [rows, K / 128], exactly as
// rlu_quant_fp8_group with group 128.
int rlu_lru_fused_quant(const int* topk_ids, int mk, int E, int S, int max_distinct,
                        int max_inserts, int* table, int* map_cold, int* slot_expert,
                        long long* slot_stamp, unsigned char* routed, long long* step, int* miss,
                        int* n_miss, int bs, int L, int NB, int* sorted_hot, int* eids_hot,
                        int* npad_hot, int* sorted_cold, int* eids_cold, int* npad_cold,
                        const void* x, int rows, int K, int ldx, void* q, float* scale,
                        hipStream_t stream) {
  if (E <= 0 || E > rlu::MAXE || S <= 0 || S > rlu::MAXS) return -1;
  if (bs <= 0 || L <= 0 || NB <= 0 || mk < 0) return -1;
  if (max_inserts < 0 || max_inserts > rlu::MAXINS) return -1;
  if (rows < 0 || K <= 0 || ldx < K || (rows > 0 && (!x || !q || !scale))) return -1;
  if (K % 128 || ldx % 8) return -2;
  const bool defer = rlu::defer_placement(mk, bs, L, NB);
  auto k = bs == 16 ? rlu::lru_k<true, 16> : rlu::lru_k<true, 0>;
  hipLaunchKernelGGL(k, dim3(1 + (rows + rlu::NW - 1) / rlu::NW), dim3(rlu::NT), 0, stream,
                     topk_ids, mk, E, S,
                     max_distinct, max_inserts, table, map_cold, slot_expert, slot_stamp,
                     routed, step, miss, n_miss, bs, L, NB, sorted_hot, eids_hot, npad_hot,
                     sorted_cold, eids_cold, npad_cold,
                     rlu::QuantJob{(const uint16_t*)x, rows, K, ldx, (uint8_t*)q, scale},
                     rlu::aligned16(sorted_hot, sorted_cold), defer);
  if (defer)
    rlu::launch_place(topk_ids, mk, E, S, table, eids_hot, eids_cold, npad_hot, npad_cold, NB,
                      bs, L, sorted_hot, sorted_cold, stream);
  return (int)hipGetLastError();
}

// kernels/lru/r4d_lru.hip:612-629
int r4d_lru_gather(void* d0, const void* s0, long b0, void* d1, const void* s1, long b1,
                   void* d2, const void* s2, long b2, void* d3, const void* s3, long b3,
                   void* d4, const void* s4, long b4, void* d5, const void* s5, long b5,
                   const int* miss, const int* n_miss, int chunks, int lanes,
                   hipStream_t stream) {
  const long bs[6] = {b0, b1, b2, b3, b4, b5};
  for (int i = 0; i < 6; i++)
    if (bs[i] <= 0 || bs[i] % 16) return -1;
  if (chunks <= 0 || lanes <= 0) return -1;
  hipLaunchKernelGGL(rlu::gather_k, dim3(chunks, lanes), dim3(rlu::NT), 0, stream,
                     (rlu::v4u*)d0, (const rlu::v4u*)s0, b0 / 16, (rlu::v4u*)d1,
                     (const rlu::v4u*)s1, b1 / 16, (rlu::v4u*)d2, (const rlu::v4u*)s2, b2 / 16,
                     (rlu::v4u*)d3, (const rlu::v4u*)s3, b3 / 16, (rlu::v4u*)d4,
                     (const rlu::v4u*)s4, b4 / 16, (rlu::v4u*)d5, (const rlu::v4u*)s5, b5 / 16,
                     miss, n_miss);
  return (int)hipGetLastError();
}

// The bucket split of the three-way overlap proposed in docs/REVIEW.md:281-301 (no kernel in
// the reference).
int rlu_lru_split_fresh(const int* eids_hot, int nb, const int* miss, const int* n_miss,
                        int miss_cap, int S, int* eids_res, int* eids_new,
                        hipStream_t stream) {
  if (nb < 0 || miss_cap < 0 || S <= 0 || S > rlu::MAXS) return -1;
  if (nb == 0) return 0;
  if (!eids_hot || !miss || !n_miss || !eids_res || !eids_new) return -1;
  hipLaunchKernelGGL(rlu::split_fresh_k, dim3(1), dim3(rlu::NT), 0, stream, eids_hot, nb, miss,
                     n_miss, miss_cap, S, eids_res, eids_new);
  return (int)hipGetLastError();
}

}  // extern "C"
