/* Serial C restatement of the device LRU expert cache -- TEST INFRASTRUCTURE ONLY.
 *
 * Built by oracle/Makefile into oracle/_build/liblru_oracle.so and loaded by oracle/clru.py.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker
 * (or as the timed CPU restatement); the product library never links it.
 *
 * It is deliberately written the "old" way, so that it pins the numpy restatement and the
 * device kernel from a different direction:
 *   - victims are taken one at a time by a linear argmin over (stamp, slot) among slots whose
 *     expert is not routed, as the pre-rewrite kernel does (kernels/lru/r4d_lru_pre_victim.hip;
 *     semantics described in kernels/lru/README.md:79-95 and tests/lru/test_lru.py:79-109);
 *   - align places tokens by walking them in index order with a per-bucket cursor (a stable
 *     counting sort), as moe_align_block_size's contract states it
 *     (tests/k1/moe_ref_harness.py:104-137).
 * Signatures mirror the C-ABI of kernels/lru/r4d_lru.hip:579-629 without the stream.
 * Return codes follow the same argument checks (-1 on a bad argument, 0 otherwise).
 */
#include <stdint.h>
#include <string.h>

#define O_MAXS 1024
#define O_MAXE 1024
#define O_MAXINS 1024

static int64_t vkey(int64_t stamp, int slot) {
  /* (stamp << 20) | slot with two's-complement wrap, as the device shift produces */
  return (int64_t)(((uint64_t)stamp << 20) | (uint64_t)(uint32_t)slot);
}

/* r4d_lru.hip:187-269 with the serial victim loop. Returns the number installed. */
static int manage_core(const int* ids, int mk, int E, int S, int max_distinct, int max_inserts,
                       int* table, int* map_cold, int* slot_expert, long long* slot_stamp,
                       unsigned char* routed, long long* step, int* miss, int* n_miss) {
  const long long st = ++step[0];
  n_miss[0] = 0;
  memset(routed, 0, (size_t)E);
  for (int i = 0; i < mk; i++)
    if (ids[i] >= 0 && ids[i] < E) routed[ids[i]] = 1;
  int distinct = 0;
  for (int e = 0; e < E; e++) distinct += routed[e];
  if (distinct > max_distinct) return 0;

  int nmiss_all = 0;
  for (int e = 0; e < E; e++) {
    if (!routed[e]) continue;
    if (table[e] >= 0) slot_stamp[table[e]] = st;
    else {
      if (nmiss_all < max_inserts) miss[2 * nmiss_all] = e;
      nmiss_all++;
    }
  }
  const int nins = nmiss_all < max_inserts ? nmiss_all : max_inserts;
  int done = 0;
  for (int r = 0; r < nins; r++) {
    int best = -1;
    int64_t bk = 0;
    for (int i = 0; i < S; i++) {
      const int ex = slot_expert[i];
      if (ex >= 0 && ex < E && routed[ex]) continue;   /* needed this step: not evictable */
      const int64_t k = vkey(slot_stamp[i], i);
      if (best < 0 || k < bk) { best = i; bk = k; }
    }
    if (best < 0) break;                               /* nothing evictable left */
    const int e = miss[2 * r];
    const int old = slot_expert[best];
    if (old >= 0) { table[old] = -1; map_cold[old] = old; }
    slot_expert[best] = e;
    slot_stamp[best] = st;
    table[e] = best;
    map_cold[e] = -1;
    miss[2 * r + 1] = best;
    done = r + 1;
  }
  n_miss[0] = done;
  return done;
}

/* stable counting-sort align of one side; bucket(t) < 0 means "not on this side" */
static void align_side(const int* bucket, int mk, int nbk, int bs, int L, int NB,
                       int* sorted_ids, int* eids, int* npad, int* cnt, int* cur) {
  memset(cnt, 0, sizeof(int) * (size_t)nbk);
  for (int t = 0; t < mk; t++)
    if (bucket[t] >= 0) cnt[bucket[t]]++;
  int run = 0;
  for (int b = 0; b < nbk; b++) {
    cur[b] = run;
    run += (cnt[b] + bs - 1) / bs * bs;
  }
  for (int i = 0; i < L; i++) sorted_ids[i] = mk;
  for (int i = 0; i < NB; i++) eids[i] = -1;
  for (int b = 0; b < nbk; b++) {
    const int blocks = (cnt[b] + bs - 1) / bs;
    for (int k = 0; k < blocks; k++)
      if (cur[b] / bs + k < NB) eids[cur[b] / bs + k] = b;
  }
  for (int t = 0; t < mk; t++) {
    const int b = bucket[t];
    if (b < 0) continue;
    if (cur[b] < L) sorted_ids[cur[b]] = t;
    cur[b]++;
  }
  npad[0] = run;
}

int oracle_lru_manage(const int* topk_ids, int mk, int E, int S, int max_distinct,
                      int max_inserts, int* table, int* map_cold, int* slot_expert,
                      long long* slot_stamp, unsigned char* routed, long long* step, int* miss,
                      int* n_miss) {
  if (E <= 0 || S <= 0 || S > O_MAXS) return -1;
  if (max_inserts < 0 || max_inserts > O_MAXINS) return -1;
  manage_core(topk_ids, mk, E, S, max_distinct, max_inserts, table, map_cold, slot_expert,
              slot_stamp, routed, step, miss, n_miss);
  return 0;
}

int oracle_lru_fused(const int* topk_ids, int mk, int E, int S, int max_distinct,
                     int max_inserts, int* table, int* map_cold, int* slot_expert,
                     long long* slot_stamp, unsigned char* routed, long long* step, int* miss,
                     int* n_miss, int bs, int L, int NB, int* sorted_hot, int* eids_hot,
                     int* npad_hot, int* sorted_cold, int* eids_cold, int* npad_cold,
                     int* scratch /* >= 2*mk + 4*1024 ints */) {
  if (E <= 0 || E > O_MAXE || S <= 0 || S > O_MAXS) return -1;
  if (bs <= 0 || L <= 0 || NB <= 0 || mk < 0) return -1;
  if (max_inserts < 0 || max_inserts > O_MAXE) return -1;
  manage_core(topk_ids, mk, E, S, max_distinct, max_inserts, table, map_cold, slot_expert,
              slot_stamp, routed, step, miss, n_miss);
  int* bh = scratch;
  int* bc = scratch + mk;
  int* cnt = scratch + 2 * mk;
  int* cur = cnt + 2048;
  for (int t = 0; t < mk; t++) {
    const int e = topk_ids[t];
    bh[t] = bc[t] = -1;
    if (e < 0 || e >= E) continue;
    const int s = table[e];
    if ((unsigned)s < (unsigned)S) bh[t] = s;
    else bc[t] = e;
  }
  align_side(bh, mk, S, bs, L, NB, sorted_hot, eids_hot, npad_hot, cnt, cur);
  align_side(bc, mk, E, bs, L, NB, sorted_cold, eids_cold, npad_cold, cnt, cur);
  return 0;
}

/* r4d_lru.hip:612-629 semantics on host memory */
int oracle_lru_gather(void* d0, const void* s0, long b0, void* d1, const void* s1, long b1,
                      void* d2, const void* s2, long b2, void* d3, const void* s3, long b3,
                      void* d4, const void* s4, long b4, void* d5, const void* s5, long b5,
                      const int* miss, const int* n_miss) {
  void* d[6] = {d0, d1, d2, d3, d4, d5};
  const void* s[6] = {s0, s1, s2, s3, s4, s5};
  const long b[6] = {b0, b1, b2, b3, b4, b5};
  for (int i = 0; i < 6; i++)
    if (b[i] <= 0 || b[i] % 16) return -1;
  for (int j = 0; j < n_miss[0]; j++) {
    const long e = miss[2 * j], sl = miss[2 * j + 1];
    for (int i = 0; i < 6; i++)
      memcpy((char*)d[i] + sl * b[i], (const char*)s[i] + e * b[i], (size_t)b[i]);
  }
  return 0;
}
