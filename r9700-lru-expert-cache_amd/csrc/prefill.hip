// The grouped fp8 GEMM of a prefill chunk (tens of rows per expert), streamed: same operands,
// row contract, tile list and numerics as tiled_k (gemm_tiled.hip) and moe_gemm_k (gemm.hip),
// bit for bit, for the K of the MoE expert shapes this library is built for (K = 2560 gate_up,
// K = 768 down; other K run tiled_k).
//
// Why a second kernel: at 80 rows per expert the work is weight streaming (about 160 FLOP per
// weight byte, under the fp8 ridge of ~625), so what matters is how many weight bytes each CU
// keeps in flight. tiled_k stages both operands through LDS one K step ahead, so a CU has one
// step (~48 KB) in flight and restarts its pipeline at every tile. Here:
//
//   * An item is (tile of <= 8 16-row blocks of one expert, 16 S W output columns). Each of the
//     W waves owns S 16-column weight strips and computes every block of the tile for them, so
//     a weight fragment is used from registers by all the tile's blocks and never goes through
//     LDS. Each wave streams its strips through a ring of D register stages (global loads,
//     nontemporal) with no barrier on them, and the ring runs on across item boundaries: the
//     last D steps of an item issue the first D steps of the next one. ~160 KB of weights are
//     in flight per CU.
//   * The tile's activation rows (gathered through sorted_ids) go to LDS in chunks of KC K
//     steps, double-buffered, loaded into registers one whole chunk ahead -- the next item's
//     first chunk during this item's last one -- and written at the chunk's end, so waiting
//     for them only waits for weight loads issued before them, which the ring needs by then
//     anyway (the vector-memory counter retires in order). One barrier per chunk.
//   * The activation scales of the chunk ride with it (LDS), the weight-block scales of an
//     item come through scalar loads, and the routed weights and row ids of the next item are
//     staged with its first chunk, so the epilogue reads LDS only. In the epilogue each wave
//     turns its own strips' bf16 outputs into 16-byte row pieces through a small LDS area of
//     its own and stores them nontemporally (the rows are scattered and not re-read here;
//     kept out of L2 they leave it to the weight stream), with no workgroup barrier, so a
//     wave that finishes early starts the next item, whose weights are already in flight.
//   * Item metadata (tile, expert) is read through scalar loads two items ahead, the next
//     tile's sorted ids one item ahead.
//   * Items go to XCDs in contiguous ranges of tiles (workgroup b runs on XCD b % 8): the
//     column groups of a tile run at the same time on CUs sharing one L2, which holds the
//     tile's rows once.
//   * One launch can cover two aligns over two weight sets (a layer's resident slots and the
//     full tensor it reads non-resident experts from): the tile list then names the set of
//     each tile (bit 16 of its block count), and an item takes its expert ids, sorted ids,
//     weights and scales from that set. Both aligns index the same activation rows and write
//     the same output.
// Per step, acc = fma(mfma(a, b), xs * ws, acc) in ascending k from zero: the same sequence of
// operations as moe_gemm_k with sk = 1, so the outputs are equal bit for bit.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_common.h"
#include "numerics.h"
#include "prefill.h"
#include "quant_row.h"
#include "wave.h"

namespace rlu {
namespace pf {

constexpr int TB = 8;           // 16-row blocks per tile: the tile list's tile size
constexpr int NXCD = 8;
constexpr int BUF_WORD3 = 0x00020000;   // raw buffer descriptor word 3 on gfx9 (no format)
constexpr int NT = 2;                   // buffer cache policy: streaming (weights are read once)

struct Args {
  const uint8_t* qx;
  const float* xs;
  const uint8_t* wq;
  const float* ws;
  const int* sorted_ids;
  const int* eids;
  const uint8_t* wq1;            // the second set (tiles with set bit 1); the first when unused
  const float* ws1;
  const int* sorted_ids1;
  const int* eids1;
  bool two;                      // a two-set tile list
  const int* tiles;
  const int* ntiles;
  uint16_t* y;
  const float* tw;
  uint8_t* q2;
  float* s2;
  int mtk;
  int top_k;
  int N;
};

struct Item {
  int b0, nbk, e, n0, set;
};

typedef unsigned v2u __attribute__((ext_vector_type(2)));


template <int NK, int W, int S, int KC, int D, int BR = 1, int BG = 2>
struct Cfg {
  static constexpr int K = NK * 128;
  static constexpr int NCH = NK / KC;            // chunks per item
  static constexpr int C = 16 * S * W;           // columns per item
  static constexpr int BPW = TB / W;             // blocks whose rows each wave stages
  static constexpr int XQ = (KC + 3) / 4;        // scale loads per lane per block and chunk
  static_assert(TB % BR == 0 && BR % BG == 0 || BG % BR == 0, "block grouping");
  static_assert(NK % KC == 0 && TB % W == 0 && D <= NK && (2 * NK) % D == 0, "config");
  // two chunks at least: a chunk-end barrier then separates an item's epilogue (LDS reads of
  // its row ids) from the writes of the row ids two items on
  static_assert(NK / KC >= 2, "at least two chunks per item");
  static_assert(S * 16 <= 128 && 128 % (S * 16) == 0, "a wave's strips share a scale block");
  // LDS: the small arrays first, then the two activation buffers, each under 64 KB so that
  // every constant offset into it fits the 16-bit offset of a ds instruction
  static constexpr int SX = 2 * KC * TB * 16;                // float [buf][ks][row]
  static constexpr int RW = 2 * TB * 16;                     // int / float [par][row]
  static constexpr int A_OFF = (SX + 2 * RW) * 4;
  static constexpr int A_BUF = TB * KC * 2 * 1024;           // [blk][ks][h][lane] x 16 B
  static_assert(A_BUF <= 65536, "an activation buffer must fit one ds offset range");
  // each wave's own epilogue staging: one block's [16 rows][S 16 columns] bf16
  static constexpr int EPI_W = 16 * S * 16 * 2;
  static constexpr int EPI_OFF = A_OFF + 2 * A_BUF;
  static constexpr size_t LDS = (size_t)EPI_OFF + W * EPI_W;
  // blocks of bf16 outputs ([16 rows][C]) one activation buffer holds in the ACT epilogue
  static constexpr int BP = A_BUF / (16 * C * 2) < TB ? A_BUF / (16 * C * 2) : TB;
  static_assert(BP >= 1, "an epilogue pass holds at least one block");
};

// ACT: the gate_up GEMM with SiLU-mul-quant in its epilogue. N = 2 I (gate | up); item g
// covers gate columns [128 g, 128 g + 128) (waves 0 .. W/2 - 1) and the matching up columns
// [I + 128 g, ...) (the other waves), so each output row's 128-column activation group is
// whole in one item. The epilogue writes q2 [mtk, I] e4m3 and s2 [mtk, I / 128] instead of y,
// computed from the bf16-rounded GEMM outputs exactly as silu_mul_quant_k computes them from
// y (same silu, product and amax reduction, same rounding).
// TWO: the tile list covers two aligns (bit 16 of a tile's block count picks the set); the
// one-set kernels take no second set, whose pointers would otherwise hold scalar registers for
// the whole launch (in the gate_up kernels the extra registers spill: +5 us on 400).
template <int NK, int W, int S, int KC, int D, int BR, int BG, bool TWT, bool ACT, bool TWO>
__global__ __launch_bounds__(W * WAVE) void stream_k(
    const uint8_t* __restrict__ qx, const float* __restrict__ xs, const uint8_t* __restrict__ wq,
    const float* __restrict__ ws, const int* __restrict__ sorted_ids,
    const int* __restrict__ eids, const uint8_t* __restrict__ wq1, const float* __restrict__ ws1,
    const int* __restrict__ sorted_ids1, const int* __restrict__ eids1,
    const int* __restrict__ tiles, const int* __restrict__ ntiles,
    uint16_t* __restrict__ y, const float* __restrict__ tw, uint8_t* __restrict__ q2,
    float* __restrict__ s2, int mtk, int top_k, int N) {
  using CF = Cfg<NK, W, S, KC, D, BR, BG>;
  constexpr int K = CF::K, NCH = CF::NCH, C = CF::C, BPW = CF::BPW, XQ = CF::XQ;
  static_assert(!ACT || (C == 256 && !TWT), "an activation item is 128 gate + 128 up columns");
  extern __shared__ __align__(16) unsigned char smem[];
  float* sx = reinterpret_cast<float*>(smem);
  int* rows = reinterpret_cast<int*>(sx + CF::SX);
  float* twl = reinterpret_cast<float*>(rows + CF::RW);

  const int lane = lane_id();
  const int w = uniform((int)(threadIdx.x / WAVE));
  const int r16 = lane & 15, c4 = lane >> 4;
  // this lane's byte address in each activation buffer, opaque to the compiler so that the
  // constant part of every fragment address stays in the instruction's offset field
  unsigned abase[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    abase[q] = CF::A_OFF + q * CF::A_BUF + lane * 16;
    asm volatile("" : "+v"(abase[q]));
  }
  auto afrag = [&](int q, int off) __attribute__((always_inline)) -> v4u {
    return *reinterpret_cast<const v4u*>(smem + abase[q] + off);
  };
  const int ncg = N / C;
  // first output column of this wave's strips in an item starting at column n0
  auto col0 = [&](int n0) __attribute__((always_inline)) -> int {
    if (!ACT) return n0 + w * S * 16;
    const int j = w * S * 16;
    return j < 128 ? n0 / 2 + j : N / 2 + n0 / 2 + j - 128;
  };
  const int nx = gridDim.x % NXCD == 0 ? NXCD : 1;
  const int xcd = (int)blockIdx.x % nx, per = (int)gridDim.x / nx;
  const int nt = ntiles[0];
  const int i1 = (int)((long long)nt * (xcd + 1) / nx) * ncg;
  const int first = (int)((long long)nt * xcd / nx) * ncg + (int)blockIdx.x / nx;
  if (first >= i1) return;
  const int cnt = (i1 - first + per - 1) / per;   // this workgroup's items: first + m * per

  auto meta = [&](int m) __attribute__((always_inline)) {
    const int it = first + (m < cnt ? m : cnt - 1) * per;
    const int ti = it / ncg;
    Item r;
    r.b0 = tiles[2 * ti];
    const int nw = tiles[2 * ti + 1];              // block count | set << 16 (TWO)
    r.nbk = TWO ? nw & 0xffff : nw;
    r.set = TWO ? nw >> 16 : 0;
    r.e = (r.set ? eids1 : eids)[r.b0];
    r.n0 = (it - ti * ncg) * C;
    return r;
  };
  // this wave's strips of an item, as a buffer: strip s, step k, half h at s 16 K + k 2048 +
  // h 1024 + lane 16 (the base and the step offset stay in scalar registers)
  auto wbase = [&](const Item& it) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(
        (void*)((it.set ? wq1 : wq) + ((size_t)it.e * N + col0(it.n0)) * K), 0, S * 16 * K,
        BUF_WORD3);
  };
  // the sorted id of row r16 of block blk of an item (mtk past the tile): one vector load,
  // issued at an item's start and used at its last chunk, so waiting for it costs nothing
  auto load_id = [&](const Item& it, int blk) __attribute__((always_inline)) {
    const bool in = blk < it.nbk;
    const int v = (it.set ? sorted_ids1 : sorted_ids)[(it.b0 + (in ? blk : 0)) * 16 + r16];
    return in ? v : mtk;
  };

  // ---- registers ----
  v4u rb[D][S][2];                    // weight ring
  v4u ra[BPW][KC][2];                 // next chunk's activation rows
  float rx[BPW][XQ];                  // ... and their scales
  float rt[BPW];                      // next item's routed weight of row r16
  int son[BPW];                       // next item's sorted id of row r16
  int arow_c[BPW], arow_n[BPW];       // activation row of row r16 (current / next item)
  bool val_c[BPW], val_n[BPW];
  int id_n[BPW];                      // next item's sorted id of row r16
  v4f acc[TB][S];

  const int voff = lane * 16;
  auto issue_b = [&](int j, __amdgpu_buffer_rsrc_t base, int k) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      rb[j][s][0] = __builtin_bit_cast(
          v4u, __builtin_amdgcn_raw_buffer_load_b128(base, voff, s * 16 * K + k * 2048, NT));
      rb[j][s][1] = __builtin_bit_cast(
          v4u, __builtin_amdgcn_raw_buffer_load_b128(base, voff + 1024, s * 16 * K + k * 2048, NT));
    }
  };
  // the rows of an item from its ids: activation row and validity of row r16 of each block
  auto rows_of = [&](const int (&id)[BPW], int (&arow)[BPW], bool (&val)[BPW],
                     int (&so_out)[BPW]) __attribute__((always_inline)) {
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi) {
      const int so = id[bi];
      so_out[bi] = so;
      val[bi] = so < mtk;
      arow[bi] = so < mtk ? so / top_k : 0;
    }
  };
  // chunk c of an item's activation rows and scales, into ra / rx; with first, also the
  // item's routed weights (rt)
  auto stage_a = [&](const int (&arow)[BPW], const bool (&val)[BPW], const int (&so)[BPW],
                     int c, bool first_chunk) __attribute__((always_inline)) {
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi) {
      const uint8_t* p = qx + (size_t)arow[bi] * K + c * KC * 128 + 16 * c4;
#pragma unroll
      for (int ks = 0; ks < KC; ++ks) {
        ra[bi][ks][0] = *reinterpret_cast<const v4u*>(p + ks * 128);
        ra[bi][ks][1] = *reinterpret_cast<const v4u*>(p + ks * 128 + 64);
      }
#pragma unroll
      for (int q = 0; q < XQ; ++q) {
        const int ks = 4 * q + c4 < KC ? 4 * q + c4 : KC - 1;
        const float v = xs[(size_t)arow[bi] * NK + c * KC + ks];
        rx[bi][q] = val[bi] ? v : 0.f;
      }
      if (TWT && first_chunk) {
        const float v = tw[val[bi] ? so[bi] : 0];
        rt[bi] = v;
      }
    }
  };
  auto write_a = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi) {
      const int blk = w + bi * W;
#pragma unroll
      for (int ks = 0; ks < KC; ++ks)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<v4u*>(smem + abase[buf] + blk * KC * 2048 + (ks * 2 + h) * 1024) =
              ra[bi][ks][h];
#pragma unroll
      for (int q = 0; q < XQ; ++q) {
        const int ks = 4 * q + c4;
        if (ks < KC) sx[(buf * KC + ks) * TB * 16 + blk * 16 + r16] = rx[bi][q];
      }
    }
  };
  auto write_rows = [&](int par) __attribute__((always_inline)) {
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi) {
      const int blk = w + bi * W;
      if (c4 == 0) {
        rows[par * TB * 16 + blk * 16 + r16] = son[bi];
        twl[par * TB * 16 + blk * 16 + r16] = TWT ? rt[bi] : 1.f;
      }
    }
  };

  // ---- prologue: item 0's first chunk, rows, scales; its first D weight steps ----
  Item mA = meta(0), mB = meta(1);
  __amdgpu_buffer_rsrc_t bcur = wbase(mA);
  __amdgpu_buffer_rsrc_t bnext = wbase(mB);
  {
    int id0[BPW];
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi) id0[bi] = load_id(mA, w + bi * W);
    rows_of(id0, arow_c, val_c, son);
#pragma unroll
    for (int j = 0; j < D; ++j) issue_b(j, bcur, j);
    stage_a(arow_c, val_c, son, 0, true);
    write_a(0);
    write_rows(0);
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi) id_n[bi] = load_id(mB, w + bi * W);
  }
  __syncthreads();

  for (int m = 0; m < cnt; m += 2) {
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      if (par == 1 && m + 1 >= cnt) break;
      const Item mC = meta(m + par + 2);
#pragma unroll
      for (int bk = 0; bk < TB; ++bk)
#pragma unroll
        for (int s = 0; s < S; ++s) acc[bk][s] = v4f{0.f, 0.f, 0.f, 0.f};
      // the weight-block scales of this wave's strips, one per step: scalar loads (they never
      // enter the vector-memory counter the weight ring waits on)
      const float* wsrow =
          (mA.set ? ws1 : ws) + ((size_t)mA.e * (N / 128) + col0(mA.n0) / 128) * NK;
      float wsr[NK];
#pragma unroll
      for (int k = 0; k < NK; ++k) wsr[k] = wsrow[k];
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int qb = (par * NCH + c) & 1;
        if (c + 1 < NCH) {
          stage_a(arow_c, val_c, son, c + 1, false);
        } else {                                    // the next item's first chunk
          rows_of(id_n, arow_n, val_n, son);
          stage_a(arow_n, val_n, son, 0, true);
        }
#pragma unroll
        for (int ks = 0; ks < KC; ++ks) {
          const int k = c * KC + ks;
          const int j = (par * NK + k) % D;
          const float wsk = wsr[k];
          v8i bf[S];
#pragma unroll
          for (int s = 0; s < S; ++s) bf[s] = pack8(rb[j][s][0], rb[j][s][1]);
          // blocks in runs of BR behind one branch on the tile's block count (a block past
          // it computes on stale rows that are never stored); scheduling fenced every BG
#pragma unroll
          for (int b0 = 0; b0 < TB; b0 += BR) {
            if (b0 < mA.nbk) {
#pragma unroll
              for (int t = 0; t < BR; ++t) {
                const int bk = b0 + t;
                const int off = (bk * KC + ks) * 2048;
                const v8i af = pack8(afrag(qb, off), afrag(qb, off + 1024));
                const v4f xr = *reinterpret_cast<const v4f*>(
                    &sx[(qb * KC + ks) * TB * 16 + bk * 16 + 4 * c4]);
                v4f f;
#pragma unroll
                for (int i = 0; i < 4; ++i) f[i] = xr[i] * wsk;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                  const v4f d = mfma_f8(af, bf[s]);
#pragma unroll
                  for (int i = 0; i < 4; ++i) acc[bk][s][i] = fmaf(d[i], f[i], acc[bk][s][i]);
                }
                if (bk % BG == BG - 1) __builtin_amdgcn_sched_barrier(0);
              }
            }
          }
          if (k + D < NK)
            issue_b(j, bcur, k + D);
          else
            issue_b(j, bnext, k + D - NK);
          // keep each step's LDS reads and MFMAs in their step (hoisting the reads of later
          // steps ahead would hold a chunk of A fragments in registers)
          __builtin_amdgcn_sched_barrier(0);
        }
        write_a(qb ^ 1);
        if (c + 1 == NCH) write_rows(par ^ 1);
        __syncthreads();
      }
      // epilogue, plain GEMM: each wave writes its own S 16 columns, block by block, through
      // its own LDS staging area -- the bf16 outputs (x routed weight) of one block as [16
      // rows][S 16], read back as 16-byte row pieces, four consecutive lanes to a row -- with
      // nontemporal stores (the rows are scattered and not re-read here; kept out of L2 they
      // leave it to the weight stream). No workgroup barrier: a wave that finishes its strips
      // goes on to the next item, whose weights its ring already holds, while the others
      // still store. The row ids and routed weights read here were written before the
      // chunk-end barrier that closed the previous item, and are rewritten only after the
      // next item's first one.
      if constexpr (!ACT) {
        uint16_t* st = reinterpret_cast<uint16_t*>(smem + CF::EPI_OFF + w * CF::EPI_W);
        const int cw = col0(mA.n0);
        constexpr int RC = S * 2;                         // 16-byte pieces per staged row
#pragma unroll
        for (int bk = 0; bk < TB; ++bk) {
          if (bk < mA.nbk) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float wt = twl[par * TB * 16 + bk * 16 + 4 * c4 + i];
#pragma unroll
              for (int s = 0; s < S; ++s)
                st[(4 * c4 + i) * S * 16 + s * 16 + r16] = f32_to_bf16(acc[bk][s][i] * wt);
            }
            wave_lds_sync();
#pragma unroll
            for (int u0 = 0; u0 < 16 * RC; u0 += WAVE) {
              const int u = u0 + lane;
              if (16 * RC % WAVE == 0 || u < 16 * RC) {
                const int rr = u / RC, ch = u - rr * RC;
                const int so = rows[par * TB * 16 + bk * 16 + rr];
                const v4u v = *reinterpret_cast<const v4u*>(st + rr * S * 16 + ch * 8);
                if (so < mtk)
                  __builtin_nontemporal_store(
                      v, reinterpret_cast<v4u*>(y + (size_t)so * N + cw + ch * 8));
              }
            }
            wave_lds_sync();
          }
        }
      } else {
        // epilogue, SiLU-mul-quant: through the activation buffer this item's last chunk used
        // (free after the chunk-end barrier) each wave puts its bf16 outputs into a [rows][C]
        // tile; then 16-lane groups take whole rows (128 gate + 128 up columns), one row each.
        // Blocks go BP at a time when the tile does not fit.
        const int qlast = (par * NCH + NCH - 1) & 1;
        uint16_t* ot = reinterpret_cast<uint16_t*>(smem + CF::A_OFF + qlast * CF::A_BUF);
#pragma unroll
        for (int p0 = 0; p0 < TB; p0 += CF::BP) {
          if (p0 < mA.nbk) {
#pragma unroll
            for (int t = 0; t < CF::BP; ++t) {
              const int bk = p0 + t;
              if (bk < TB && bk < mA.nbk) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  const int rr = t * 16 + 4 * c4 + i;
#pragma unroll
                  for (int s = 0; s < S; ++s)
                    ot[rr * C + (w * S + s) * 16 + r16] = f32_to_bf16_hw(acc[bk][s][i]);
                }
              }
            }
            __syncthreads();
            const int nr = ((mA.nbk < p0 + CF::BP ? mA.nbk : p0 + CF::BP) - p0) * 16;
            // one 16-lane row group per output row, lane l on columns [8 l, 8 l + 8) of the
            // item's 128-column group (nr is a multiple of 16, so every wave's four groups
            // run the same trip count and the DPP reduction sees whole groups)
            const int I = N / 2, g = mA.n0 / C, l16 = lane & 15;
            for (int rr = (int)threadIdx.x / 16; rr < nr; rr += W * 4) {
              float gv[8], uv[8], a[8];
              unpack8_bf16(*reinterpret_cast<const uint4*>(ot + rr * C + 8 * l16), gv);
              unpack8_bf16(*reinterpret_cast<const uint4*>(ot + rr * C + 128 + 8 * l16), uv);
              uint32_t mx = 0;
#pragma unroll
              for (int j = 0; j < 8; ++j) {
                a[j] = bf16_to_f32(f32_to_bf16_hw(__fmul_rn(silu_bf16_hw(gv[j]), uv[j])));
                mx = max(mx, abs_bits(a[j]));
              }
              const float sc = scale_of(row_max_u32(mx));
              const uint2 qv = quant8(a, sc);
              const int so = rows[par * TB * 16 + p0 * 16 + rr];
              if (so < mtk) {
                __builtin_nontemporal_store(
                    v2u{qv.x, qv.y},
                    reinterpret_cast<v2u*>(q2 + (size_t)so * I + g * 128 + 8 * l16));
                if (l16 == 0) __builtin_nontemporal_store(sc, s2 + (size_t)so * (I / 128) + g);
              }
            }
            __syncthreads();
          }
        }
      }
      // advance: the next item becomes current
#pragma unroll
      for (int bi = 0; bi < BPW; ++bi) {
        arow_c[bi] = arow_n[bi];
        val_c[bi] = val_n[bi];
      }
      mA = mB;
      mB = mC;
      bcur = bnext;
      bnext = wbase(mB);
#pragma unroll
      for (int bi = 0; bi < BPW; ++bi) id_n[bi] = load_id(mB, w + bi * W);
    }
  }
}

// ACT_CFG: the configuration of the SiLU-mul-quant variant (built only for it), else of the
// plain kernels
template <int NK, int W, int S, int KC, int D, bool ACT_CFG = false, int BR = 1, int BG = 2,
          int OCC = 1>
static int launch_cfg(const Args& a, int max_tiles, hipStream_t stream) {
  using CF = Cfg<NK, W, S, KC, D, BR, BG>;
  if (a.N % CF::C) return -1;
  if ((a.q2 != nullptr) != ACT_CFG || (a.q2 && (a.tw || CF::C != 256))) return -1;
  const int items = max_tiles * (a.N / CF::C);
  int grid = device_cus() * OCC;
  if (grid > items) grid = items;
  if (grid >= NXCD) grid -= grid % NXCD;
#define RLU_PF1(T, A, TW)                                                                     \
  hipLaunchKernelGGL((stream_k<NK, W, S, KC, D, BR, BG, T, A, TW>), dim3(grid), dim3(W * WAVE), \
                     CF::LDS, stream, a.qx, a.xs, a.wq, a.ws, a.sorted_ids, a.eids, a.wq1,      \
                     a.ws1, a.sorted_ids1, a.eids1, a.tiles, a.ntiles, a.y, a.tw, a.q2, a.s2,   \
                     a.mtk, a.top_k, a.N)
#define RLU_PF(T, A)                                                                          \
  do {                                                                                        \
    if (a.two)                                                                                \
      RLU_PF1(T, A, true);                                                                    \
    else                                                                                      \
      RLU_PF1(T, A, false);                                                                   \
  } while (0)
  if constexpr (ACT_CFG)
    RLU_PF(false, true);
  else if (a.tw)
    RLU_PF(true, false);
  else
    RLU_PF(false, false);
#undef RLU_PF
#undef RLU_PF1
  return 0;
}

}  // namespace pf

// the kernel arguments; without a second set, set 1 repeats set 0 (no tile names it)
static pf::Args make_args(const void* qx, const float* xs, const void* wq, const float* ws,
                          const int* sorted_ids, const int* expert_ids, const PfSecond* second,
                          const int* tiles, const int* ntiles, const float* topk_weights,
                          void* y, void* q2, float* s2, int mtk, int top_k, int N) {
  const PfSecond one{wq, ws, sorted_ids, expert_ids};
  const PfSecond& b = second ? *second : one;
  return pf::Args{(const uint8_t*)qx, xs, (const uint8_t*)wq, ws, sorted_ids, expert_ids,
                  (const uint8_t*)b.wq, b.ws, b.sorted_ids, b.expert_ids, second != nullptr,
                  tiles, ntiles,
                  (uint16_t*)y, topk_weights, (uint8_t*)q2, s2, mtk, top_k, N};
}

bool prefill_stream_built(int K, int N) { return (K == 2560 || K == 768) && N % 256 == 0; }

int launch_prefill_stream(const void* qx, const float* xs, const void* wq, const float* ws,
                          const int* sorted_ids, const int* expert_ids, const PfSecond* second,
                          const int* tiles, const int* ntiles, int max_tiles,
                          const float* topk_weights, void* y, int mtk, int top_k, int K, int N,
                          hipStream_t stream) {
  const pf::Args a = make_args(qx, xs, wq, ws, sorted_ids, expert_ids, second, tiles, ntiles,
                               topk_weights, y, nullptr, nullptr, mtk, top_k, N);
  if (K == 2560) return pf::launch_cfg<20, 8, 2, 4, 5>(a, max_tiles, stream);
  if (K == 768) return pf::launch_cfg<6, 8, 2, 3, 6>(a, max_tiles, stream);
  return -1;
}

bool prefill_stream_act_built(int K, int N) { return K == 2560 && N % 256 == 0; }

int launch_prefill_stream_act(const void* qx, const float* xs, const void* wq, const float* ws,
                              const int* sorted_ids, const int* expert_ids,
                              const PfSecond* second, const int* tiles, const int* ntiles,
                              int max_tiles, void* q2, float* s2, int mtk, int top_k, int K,
                              int N, hipStream_t stream) {
  const pf::Args a = make_args(qx, xs, wq, ws, sorted_ids, expert_ids, second, tiles, ntiles,
                               nullptr, nullptr, q2, s2, mtk, top_k, N);
  if (K == 2560) return pf::launch_cfg<20, 8, 2, 4, 4, true>(a, max_tiles, stream);
  return -1;
}

}  // namespace rlu
