// Channel-given selected contraction on gfx950 (the numerator-only read of
// the feature-mass writers, indirect_fine.py:65-133 and its backward
// :101-120, :172-227):
//   out[b, q, h, e]  = bf16(sum_m sum_d channel[b, q, h, m, d] C[id_m][d][e])
//   d channel[.., m, d] = bf16(sum_e grad[b, q, h, e] C[id_m][d][e])
//   d C[bb, h, s]    = bf16(sum over b % BB == bb of bf16(sum over the pairs
//                      (q, m) of batch b with id_m == s of channel^T grad))
// C rows d, columns e; batch b reads bank b % BB.
//
// The reference sorts every (query, slot) pair by fine id and runs one C tile
// per fine against 32 pairs at a time, then sums the pairs of a query. Here a
// workgroup owns a tile of queries of one (b, h) instead: the union of the
// tile's selected ids (an LDS bitmask, ascending) is walked once, each fine's
// C is staged in LDS once (the next fine's C and channel rows are loaded
// while the current one runs) and every wave builds its MFMA A operand from
// the channel rows of the queries that selected that fine (zero rows elsewhere),
// so the numerator accumulates in one v_mfma_f32_32x32x16_bf16 accumulator
// per (32 queries, 32 columns) and no pair buffer or sort is needed. A query
// that lists one fine twice is handled exactly by one pass per occurrence.
// The fp32 sum runs in fine order inside the MFMA instead of slot order, a
// difference at fp32 rounding before the final bf16 cast.
#include "tao_launch.h"
#include "tao_common.h"

namespace tao {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

TAO_DEV bf16x8 as_bf16x8(const uint4& u) {
  bf16x8 r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

constexpr int kSelThreads = 256;
constexpr int kSelMaxM = 64;
constexpr int kSelMaxS = 4096;
constexpr int kSelWords = kSelMaxS / 32;

template <int D> constexpr int kSelQG = 128 / D;          // 32-query groups per tile
template <int D> constexpr int kSelTileQ = 32 * kSelQG<D>;
// The forward's tile: each wave owns 32 queries and every column of them,
// so a staged C^T serves kSelThreads / 64 * 32 queries.
constexpr int kSelFwdQ = 32 * (kSelThreads / 64);

template <int D, int TQ = kSelTileQ<D>, bool STAGE = true>
struct SelSmem {
  static constexpr int kUni = TQ * kSelMaxM < kSelMaxS ? TQ * kSelMaxM : kSelMaxS;
  bf16_t c[D][D + 8];                     // staged C^T (forward) or C (grad of channel)
  int16_t sid[TQ][kSelMaxM];              // the tile's selected ids
  int8_t occ[TQ][kSelMaxM];               // occurrence index of sid[q][m] in its row
  uint32_t bits[kSelWords];
  int pre[kSelWords];
  int16_t uni[kUni];                      // the union: at most S and TQ * M ids (S < 2^15)
  int8_t ord[TQ][kSelMaxM];               // forward: a row's slots by (id, slot) ascending
  int n_union, passes;
  bf16_t stage[STAGE ? 4 : 1][32][40];    // grad-of-channel rows per wave (32 q x 32 d)
};

// Shared setup: ids of the tile into LDS, occurrence indices, the union
// (ascending) and the number of passes (largest occurrence count).
template <typename Smem>
TAO_DEV void tile_union(Smem& sm, const SelectedParams& p, int b, int h, int q0, int nq,
                        int tid) {
  for (int i = tid; i < kSelWords; i += kSelThreads) sm.bits[i] = 0u;
  if (tid == 0) sm.passes = 0;
  __syncthreads();
  for (int i = tid; i < nq * p.M; i += kSelThreads) {
    const int q = i / p.M, m = i % p.M;
    const int64_t id64 = p.ids[(((size_t)b * p.Q + q0 + q) * p.H + h) * p.M + m];
    const bool ok = id64 >= 0 && id64 < p.S;        // an id outside the bank reads nothing
    const int id = ok ? (int)id64 : -1;
    sm.sid[q][m] = (int16_t)id;
    if (ok) atomicOr(&sm.bits[id >> 5], 1u << (id & 31));
  }
  __syncthreads();
  for (int i = tid; i < nq * p.M; i += kSelThreads) {
    const int q = i / p.M, m = i % p.M;
    const int id = sm.sid[q][m];
    int o = 0;
    for (int j = 0; j < m; ++j) o += sm.sid[q][j] == id;
    sm.occ[q][m] = (int8_t)o;
    if (o) atomicMax(&sm.passes, o);
  }
  if (tid < 64) {
    constexpr int WPL = kSelWords / 64;
    int cnt[WPL], total = 0;
#pragma unroll
    for (int i = 0; i < WPL; ++i) { cnt[i] = __popc(sm.bits[tid * WPL + i]); total += cnt[i]; }
    int incl = total;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off, 64);
      if (tid >= off) incl += v;
    }
    int run = incl - total;
#pragma unroll
    for (int i = 0; i < WPL; ++i) { sm.pre[tid * WPL + i] = run; run += cnt[i]; }
    if (tid == 63) sm.n_union = incl;
  }
  __syncthreads();
  for (int i = tid; i < kSelWords; i += kSelThreads) {
    uint32_t bits = sm.bits[i];
    int r = sm.pre[i];
    while (bits) {
      sm.uni[r++] = (int16_t)(i * 32 + __ffs(bits) - 1);
      bits &= bits - 1;
    }
  }
  __syncthreads();
}

// Slot of fine f (occurrence r) in query row q, or -1.
template <typename Smem>
TAO_DEV int find_slot(const Smem& sm, int q, int M, int f, int r) {
  for (int m = 0; m < M; ++m)
    if (sm.sid[q][m] == f && sm.occ[q][m] == r) return m;
  return -1;
}

template <int D>
__global__ __launch_bounds__(kSelThreads, 2) void selected_fwd_kernel(SelectedParams p) {
  constexpr int KK = D / 16, ET = D / 32, TQ = kSelFwdQ;
  constexpr int CPR = D / 8;                             // uint4 per row of C
  constexpr int PJ = (D / 2) * CPR / kSelThreads;        // row-pair jobs per thread
  static_assert(PJ * kSelThreads == (D / 2) * CPR, "whole row-pair jobs");
  __shared__ SelSmem<D, TQ, false> sm;
  const int n_tiles = (p.Q + TQ - 1) / TQ;
  const int tile = blockIdx.x % n_tiles, bh = blockIdx.x / n_tiles;
  const int b = bh / p.H, h = bh % p.H;
  const int q0 = tile * TQ, nq = min(TQ, p.Q - q0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  tile_union(sm, p, b, h, q0, nq, tid);
  // Each row's slots in ascending (id, slot) order: the union is walked in
  // ascending id, so a lane finds its query's slots of fine f at a pointer
  // (invalid ids sort first and are skipped).
  for (int q = tid; q < nq; q += kSelThreads) {
    for (int i = 0; i < p.M; ++i) sm.ord[q][i] = (int8_t)i;
    for (int i = 1; i < p.M; ++i) {
      const int8_t m = sm.ord[q][i];
      const int key = sm.sid[q][m];
      int j = i - 1;
      while (j >= 0 && sm.sid[q][sm.ord[q][j]] > key) { sm.ord[q][j + 1] = sm.ord[q][j]; --j; }
      sm.ord[q][j + 1] = m;
    }
  }
  __syncthreads();
  const int U = sm.n_union;
  const int ql = 32 * w + li;                             // the lane's query row in the tile
  const bool qok = ql < nq;
  int ptr = 0;
  if (qok)
    while (ptr < p.M && sm.sid[ql][sm.ord[ql][ptr]] < 0) ++ptr;
  // Next slot of fine f in this lane's row, or -1.
  auto next_slot = [&](int f) __attribute__((always_inline)) {
    if (!qok || ptr >= p.M) return -1;
    const int m = sm.ord[ql][ptr];
    if (sm.sid[ql][m] != f) return -1;
    ++ptr;
    return m;
  };
  const bf16_t* chan = p.channel + (((size_t)b * p.Q + q0 + (qok ? ql : 0)) * p.H + h) * p.M * D;
  auto load_row = [&](int m, uint4 (&r)[KK]) __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      r[kk] = m >= 0 ? *(const uint4*)(chan + (size_t)m * D + 16 * kk + 8 * hl)
                     : make_uint4(0u, 0u, 0u, 0u);
  };
  const bf16_t* bank = p.bank + ((size_t)(b % p.BB) * p.H + h) * p.S * D * D;
  // C of a fine into registers: job j = row pair d = 2 (j % (D / 2)), chunk
  // j / (D / 2), so consecutive threads write consecutive words of a C^T row.
  uint4 c0[PJ], c1[PJ];
  auto load_c = [&](int f) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int job = tid + j * kSelThreads;
      const int d = 2 * (job % (D / 2)), e0 = 8 * (job / (D / 2));
      const bf16_t* src = bank + (size_t)f * D * D + (size_t)d * D + e0;
      c0[j] = *(const uint4*)src;
      c1[j] = *(const uint4*)(src + D);
    }
  };
  floatx16 acc[ET];
#pragma unroll
  for (int t = 0; t < ET; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
  int m_next = -1;
  uint4 row_next[KK];
  if (U > 0) {
    load_c(sm.uni[0]);
    m_next = next_slot(sm.uni[0]);
    load_row(m_next, row_next);
  }
  for (int u = 0; u < U; ++u) {
    const int f = sm.uni[u];
    __syncthreads();                                     // previous fine consumed
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int job = tid + j * kSelThreads;
      const int d = 2 * (job % (D / 2)), e0 = 8 * (job / (D / 2));
      const uint32_t a[4] = {c0[j].x, c0[j].y, c0[j].z, c0[j].w};
      const uint32_t bq[4] = {c1[j].x, c1[j].y, c1[j].z, c1[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *(uint32_t*)&sm.c[e0 + 2 * i][d] = (a[i] & 0xFFFFu) | (bq[i] << 16);
        *(uint32_t*)&sm.c[e0 + 2 * i + 1][d] = (a[i] >> 16) | (bq[i] & 0xFFFF0000u);
      }
    }
    __syncthreads();
    if (u + 1 < U) load_c(sm.uni[u + 1]);                // in flight during this fine's MFMAs
    int m = m_next;
    uint4 row[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) row[kk] = row_next[kk];
    // Every slot of f in the lane's row (a fine listed twice adds twice).
    while (__any(m >= 0)) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
#pragma unroll
        for (int et = 0; et < ET; ++et)
          acc[et] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              as_bf16x8(row[kk]),
              as_bf16x8(*(const uint4*)&sm.c[32 * et + li][16 * kk + 8 * hl]), acc[et], 0, 0, 0);
      m = m >= 0 ? next_slot(f) : -1;
      load_row(m, row);
    }
    if (u + 1 < U) {
      m_next = next_slot(sm.uni[u + 1]);
      load_row(m_next, row_next);
    }
  }
  // rows q = 32 w + 8 (i / 4) + 4 hl + i % 4, column e = 32 et + li
#pragma unroll
  for (int et = 0; et < ET; ++et)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int q = 32 * w + 8 * (i / 4) + 4 * hl + (i % 4);
      if (q < nq)
        p.out[(((size_t)b * p.Q + q0 + q) * p.H + h) * D + 32 * et + li] = f2bf(acc[et][i]);
    }
}

// d channel: A = the tile's grad rows (loaded once), B = rows of C (k = e).
template <int D>
__global__ __launch_bounds__(kSelThreads) void selected_bwd_a_kernel(SelectedParams p) {
  constexpr int KK = D / 16, ET = D / 32, TQ = kSelTileQ<D>;
  constexpr int CJ = D * D / 8 / kSelThreads;
  __shared__ SelSmem<D> sm;
  const int n_tiles = (p.Q + TQ - 1) / TQ;
  const int tile = blockIdx.x % n_tiles, bh = blockIdx.x / n_tiles;
  const int b = bh / p.H, h = bh % p.H;
  const int q0 = tile * TQ, nq = min(TQ, p.Q - q0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const int qg = w / ET, dt = w % ET;
  tile_union(sm, p, b, h, q0, nq, tid);
  const int U = sm.n_union, R = sm.passes + 1;
  const int ql = 32 * qg + li;
  const bool qok = ql < nq;
  const bf16_t* bank = p.bank + ((size_t)(b % p.BB) * p.H + h) * p.S * D * D;
  uint4 ga[KK];
  {
    const bf16_t* grow = p.grad + (((size_t)b * p.Q + q0 + (qok ? ql : 0)) * p.H + h) * D;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      ga[kk] = qok ? *(const uint4*)(grow + 16 * kk + 8 * hl) : make_uint4(0, 0, 0, 0);
  }
  // slots whose id lies outside the bank read nothing: zero gradient
  if (qok)
    for (int m = 0; m < p.M; ++m)
      if (sm.sid[ql][m] < 0) {
        bf16_t* dst = p.grad_channel +
            ((((size_t)b * p.Q + q0 + ql) * p.H + h) * p.M + m) * D + 32 * dt + 16 * hl;
        *(uint4*)dst = make_uint4(0, 0, 0, 0);
        *(uint4*)(dst + 8) = make_uint4(0, 0, 0, 0);
      }
  for (int u = 0; u < U; ++u) {
    const int f = sm.uni[u];
    uint32_t cw[CJ][4];
#pragma unroll
    for (int j = 0; j < CJ; ++j) {
      const uint4 v = *(const uint4*)(bank + (size_t)f * D * D + (size_t)(tid + j * kSelThreads) * 8);
      cw[j][0] = v.x; cw[j][1] = v.y; cw[j][2] = v.z; cw[j][3] = v.w;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < CJ; ++j) {
      const int idx = (tid + j * kSelThreads) * 8;
      *(uint4*)&sm.c[idx / D][idx % D] = make_uint4(cw[j][0], cw[j][1], cw[j][2], cw[j][3]);
    }
    __syncthreads();
    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          as_bf16x8(ga[kk]), as_bf16x8(*(const uint4*)&sm.c[32 * dt + li][16 * kk + 8 * hl]), acc,
          0, 0, 0);
    // through the wave's LDS stage: row q = li, 16 columns per half-wave
#pragma unroll
    for (int i = 0; i < 16; ++i) sm.stage[w][8 * (i / 4) + 4 * hl + (i % 4)][li] = f2bf(acc[i]);
    __syncthreads();
    if (qok) {
      const uint4 lo = *(const uint4*)&sm.stage[w][li][16 * hl];
      const uint4 hi = *(const uint4*)&sm.stage[w][li][16 * hl + 8];
      for (int r = 0; r < R; ++r) {
        const int m = find_slot(sm, ql, p.M, f, r);
        if (m < 0) continue;
        bf16_t* dst = p.grad_channel +
            ((((size_t)b * p.Q + q0 + ql) * p.H + h) * p.M + m) * D + 32 * dt + 16 * hl;
        *(uint4*)dst = lo;
        *(uint4*)(dst + 8) = hi;
      }
    }
  }
}

// d C: one workgroup per (bank batch bb, head, NF consecutive fines); for each
// batch b = bb, bb + BB, ... the pairs of b are reduced in fp32 (k = query,
// 32 at a time, channel^T and grad^T staged transposed), rounded to bf16 and
// added to the running total.
template <int D> constexpr int kSelNF = D == 64 ? 4 : 1;

template <int D>
__global__ __launch_bounds__(kSelThreads) void selected_bwd_c_kernel(SelectedParams p) {
  constexpr int NF = kSelNF<D>, DT = D / 32, NT = NF * DT * DT, TPW = NT / 4;
  __shared__ bf16_t cht[NF][D][40], gt[D][40];
  __shared__ uint64_t match[NF][32];
  __shared__ int any_sel[NF];
  const int groups = (p.S + NF - 1) / NF;
  const int g = blockIdx.x % groups, bbh = blockIdx.x / groups;
  const int bb = bbh / p.H, h = bbh % p.H;
  const int f0 = g * NF;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  floatx16 acc[TPW], total[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) { acc[j][i] = 0.0f; total[j][i] = 0.0f; }
  for (int b = bb; b < p.B; b += p.BB) {
    for (int qb = 0; qb < p.Q; qb += 32) {
      __syncthreads();
      if (tid < NF) any_sel[tid] = 0;
      if (tid < 32) {
        uint64_t mk[NF];
#pragma unroll
        for (int k = 0; k < NF; ++k) mk[k] = 0;
        if (qb + tid < p.Q) {
          const int64_t* ids = p.ids + (((size_t)b * p.Q + qb + tid) * p.H + h) * p.M;
          for (int m = 0; m < p.M; ++m) {
            const int64_t k = ids[m] - f0;
#pragma unroll
            for (int kk = 0; kk < NF; ++kk)
              if (k == kk) mk[kk] |= 1ull << m;
          }
        }
#pragma unroll
        for (int k = 0; k < NF; ++k) match[k][tid] = mk[k];
      }
      __syncthreads();
      // thread = (query qi, 8-channel chunk c)
      for (int job = tid; job < 32 * (D / 8); job += kSelThreads) {
        const int qi = job % 32, c = job / 32;
        const int q = qb + qi;
        const bool qok = q < p.Q;
        const size_t row = ((size_t)b * p.Q + (qok ? q : 0)) * p.H + h;
        const uint4 gv = qok ? *(const uint4*)(p.grad + row * D + 8 * c) : make_uint4(0, 0, 0, 0);
        const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          gt[8 * c + 2 * j][qi] = (bf16_t)(gw[j] & 0xFFFFu);
          gt[8 * c + 2 * j + 1][qi] = (bf16_t)(gw[j] >> 16);
        }
#pragma unroll
        for (int k = 0; k < NF; ++k) {
          uint64_t mk = match[k][qi];
          float sv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) sv[j] = 0.0f;
          if (mk && c == 0) any_sel[k] = 1;
          while (mk) {
            const int m = __builtin_ctzll(mk);
            mk &= mk - 1;
            const uint4 cvv = *(const uint4*)(p.channel + (row * p.M + m) * D + 8 * c);
            const uint32_t cw[4] = {cvv.x, cvv.y, cvv.z, cvv.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              sv[2 * j] += __uint_as_float(cw[j] << 16);
              sv[2 * j + 1] += __uint_as_float(cw[j] & 0xFFFF0000u);
            }
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) cht[k][8 * c + j][qi] = f2bf(sv[j]);
        }
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int tt = w + 4 * j;
        const int k = tt / (DT * DT), r = tt % (DT * DT);
        const int mt = r / DT, nt = r % DT;
        if (!any_sel[k]) continue;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              as_bf16x8(*(const uint4*)&cht[k][32 * mt + li][16 * ks + 8 * hl]),
              as_bf16x8(*(const uint4*)&gt[32 * nt + li][16 * ks + 8 * hl]), acc[j], 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        total[j][i] += rbf(acc[j][i]);
        acc[j][i] = 0.0f;
      }
  }
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int tt = w + 4 * j;
    const int k = tt / (DT * DT), r = tt % (DT * DT);
    const int mt = r / DT, nt = r % DT;
    const int f = f0 + k;
    if (f >= p.S) continue;
    bf16_t* out = p.grad_bank + (((size_t)bb * p.H + h) * p.S + f) * D * D;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = 32 * mt + 8 * (i / 4) + 4 * hl + (i % 4);
      out[(size_t)d * D + 32 * nt + li] = f2bf(total[j][i]);
    }
  }
}

}  // namespace

hipError_t launch_selected_numerator(const SelectedParams& p, int head_dim, hipStream_t s) {
  if (p.M > kSelMaxM || p.S > kSelMaxS || p.S > 32767) return hipErrorInvalidValue;
  if (p.B * p.Q * p.H == 0) return hipSuccess;
#define TAO_SEL_FWD(D_)                                                                       \
  hipLaunchKernelGGL(selected_fwd_kernel<D_>,                                                 \
                     dim3((unsigned)(((p.Q + kSelFwdQ - 1) / kSelFwdQ) * p.B * p.H)),        \
                     dim3(kSelThreads), 0, s, p)
  if (head_dim == 128)
    TAO_SEL_FWD(128);
  else if (head_dim == 64)
    TAO_SEL_FWD(64);
  else
    return hipErrorInvalidValue;
#undef TAO_SEL_FWD
  return hipGetLastError();
}

hipError_t launch_selected_numerator_bwd(const SelectedParams& p, int head_dim, hipStream_t s) {
  if (p.M > kSelMaxM || p.S > kSelMaxS || p.S > 32767) return hipErrorInvalidValue;
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
#define TAO_SEL_BWD(D_)                                                                         \
  do {                                                                                          \
    if (p.grad_channel && p.B * p.Q * p.H > 0)                                                  \
      hipLaunchKernelGGL(selected_bwd_a_kernel<D_>,                                             \
                         dim3((unsigned)(((p.Q + kSelTileQ<D_> - 1) / kSelTileQ<D_>) * p.B *    \
                                         p.H)),                                                 \
                         dim3(kSelThreads), 0, s, p);                                           \
    if (p.grad_bank && p.BB * p.H * p.S > 0)                                                    \
      hipLaunchKernelGGL(selected_bwd_c_kernel<D_>,                                             \
                         dim3((unsigned)(((p.S + kSelNF<D_> - 1) / kSelNF<D_>) * p.BB * p.H)),  \
                         dim3(kSelThreads), 0, s, p);                                           \
  } while (0)
  if (head_dim == 128)
    TAO_SEL_BWD(128);
  else
    TAO_SEL_BWD(64);
#undef TAO_SEL_BWD
  return hipGetLastError();
}

}  // namespace tao
