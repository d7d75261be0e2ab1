// Batched prefill kernels for gfx950: the page / epoch bookkeeping of every
// seal in a prompt and the selected fine read of every query.
//
// A prompt seals many fines. The reference reads each chunk against the
// state left by the previous chunk's seal (tao_stream.py:919-969); here every
// seal epoch's page weights and pending segment weights are materialised in
// pools at once (pages_kernel + epochs_kernel), routes for all refresh turns
// run in one launch (route.hip, turn mode), and read_tiles_kernel performs
// the selected read + fusion of all queries.
//
// read_groups_kernel: the selected read + fusion of every query, one
// workgroup per 8 read tiles (route turns) of one head; see the kernel.
#include "tao_launch.h"
#include "tao_common.h"
#include "tao_fusion.h"

namespace tao {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kTileQ = 32;
constexpr int kMaxM = 128;
constexpr int kMaxFineIds = 16384;   // fine ids a turn-group read can index

TAO_DEV bf16x8 as_bf16x8(const uint4& u) {
  bf16x8 r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

template <int D>
__global__ __launch_bounds__(kThreads) void pages_kernel(PagesParams p) {
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int g = p.first_page + blockIdx.x / BH;
  const int d = threadIdx.x;
  if (d >= D) return;
  const bf16_t* z = p.fine_z + (size_t)bh * p.fine_cap * D;
  float zv[8];
  for (int i = 0; i < 8; ++i) zv[i] = bf2f(z[(size_t)(g * p.group + i) * D + d]);
  const float pz = group_logsumexp(zv, 8);
  p.page_z[((size_t)bh * p.page_cap + g) * D + d] = f2bf(pz);
  for (int i = 0; i < 8; ++i)
    p.fine_sw[((size_t)bh * p.fine_cap + g * p.group + i) * D + d] = f2bf(exp_bf(rbf(zv[i] - pz)));
}

// One workgroup per (epoch, batch, head): the pending page summary with one
// thread per channel, then the page weights with one wave per channel.
template <int D>
__global__ __launch_bounds__(kThreads) void epochs_kernel(EpochParams p) {
  __shared__ float pend_pz[D];
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int erel = blockIdx.x / BH;
  const int epoch = p.first_epoch + erel;
  const bool last = erel == p.count - 1;
  const int K = epoch / p.group, pend = epoch % p.group;
  const int P = K + (pend > 0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bf16_t* z = p.fine_z + (size_t)bh * p.fine_cap * D;
  bf16_t* psw = p.psw_pool + ((size_t)erel * BH + bh) * 8 * D;
  bf16_t* pw = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
  if (tid < D && pend > 0) {
    float zv[8];
    for (int i = 0; i < 8; ++i) zv[i] = i < pend ? bf2f(z[(size_t)(K * p.group + i) * D + tid]) : 0.0f;
    const float pz = group_logsumexp(zv, pend);
    pend_pz[tid] = pz;
    for (int i = 0; i < pend; ++i) {
      const bf16_t w = f2bf(exp_bf(rbf(zv[i] - pz)));
      psw[(size_t)i * D + tid] = w;
      if (last) p.fine_sw[((size_t)bh * p.fine_cap + K * p.group + i) * D + tid] = w;
    }
    if (last) p.page_z[((size_t)bh * p.page_cap + K) * D + tid] = f2bf(pz);
  }
  __syncthreads();
  if (P == 0) return;
  const bf16_t* pzg = p.page_z + (size_t)bh * p.page_cap * D;
  bf16_t* state_pw = p.page_w + (size_t)bh * p.page_cap * D;
  for (int d = wave; d < D; d += kThreads / 64) {
    page_weights_wave(
        lane, P,
        [&](int pg) { return pg == K ? pend_pz[d] : bf2f(pzg[(size_t)pg * D + d]); },
        [&](int pg, bf16_t w) {
          pw[(size_t)pg * D + d] = w;
          if (last) state_pw[(size_t)pg * D + d] = w;
        });
  }
}

// Turn-group read: one 512-thread workgroup per (8 consecutive read tiles,
// batch, head); wave w owns tile w (<= 32 queries sharing one route, its
// own seal epoch and segment-weight source). The workgroup reads each fine
// of the union of the 8 selected sets once: C^T is staged into padded LDS
// (double-buffered, the next fine's rows in flight in registers), and every
// wave whose tile selected that fine builds its A operand
//   ch[q][d] = r(r(h_q[d] * pw[page][d]) * sw[fine][d])
// in registers (MFMA A layout; r(h * pw) is kept per page) and runs
// 4 x 8 v_mfma_f32_32x32x16_bf16 into its 32 x D accumulator, plus one
// against a column of ones for den[q] = sum over the tile's fines of
// sum_d ch; fine = r(r(num) / r(den)), then the fusion epilogue. With the
// coarse value branch (COARSE), each e-tile of a tile whose chunk has
// completed pages also runs 8 MFMAs of the wave's h against the folded
// coarse matrix of its page count (coarse.hip) before the fusion.
//
// PERQ (the full-sequence read, every query routed by itself): selections
// are per-query bitmasks (route_queries_kernel). The union and the per-wave
// masks come from the OR of the wave's bitmasks, and each A row is zeroed
// unless its own query selected the fine, so a wave's 32 queries still share
// every staged C^T and MFMA; the numerator and denominator of a query sum
// exactly its selected fines (selected_read.py:156-173).
constexpr int kGroupWaves = 8;
constexpr int kGroupThreads = 64 * kGroupWaves;
constexpr int kBitWords = kMaxFineIds / 32;
constexpr int kMaxUnion = kGroupWaves * kMaxM;

template <int D>
struct GroupSmem {
  union {
    struct {
      uint32_t bits[kBitWords];
      int pre[kBitWords];
      uint32_t wbits[kGroupWaves][kBitWords];   // PERQ: OR of each wave's bitmasks
    } setup;
    bf16_t c[2][D][D + 8];        // staged C^T, rows padded by 16 bytes
  } u;
  bf16_t pwsw[kGroupWaves][2][2][D];   // per wave, per buffer: pw row, sw row
  bf16_t hq[kGroupWaves][32][D + 8];   // per wave: h of its queries (bf16, padded rows)
  int ids[kGroupWaves][kMaxM];
  int uni[kMaxUnion];
  uint32_t mask[kMaxUnion / 4];        // byte u: bit w set if wave w selected uni[u]
  int n_union;
};

TAO_DEV void unpack8f(const uint4& u, float out[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

template <int D, bool COARSE, bool PERQ>
__global__ __launch_bounds__(kGroupThreads) void read_groups_kernel(ReadTilesParams p) {
  constexpr int KK = D / 16, ET = D / 32, CPR = D / 8;   // k-steps, e-tiles, uint4 per row
  constexpr int CPT = D * CPR / kGroupThreads;           // C^T uint4 per thread
  __shared__ GroupSmem<D> sm;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int grp = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const int t0 = grp * kGroupWaves;
  const int nt = min(kGroupWaves, p.n_tiles - t0);

  // This wave's tile.
  int q_first = 0, nq = 0, slot = 0, M = 0, erel = 0, sw_split = 0, fine_on = 0, cpages = 0;
  if (w < nt) {
    const int64_t* desc = p.tiles + 8 * (t0 + w);
    q_first = (int)desc[0]; nq = (int)desc[1]; slot = (int)desc[2]; M = (int)desc[3];
    erel = (int)desc[4]; sw_split = (int)desc[5]; fine_on = (int)desc[6];
    cpages = (int)desc[7];
  }
  const bool reads = w < nt && fine_on;
  if (w < nt && !fine_on) {
    // Before the first seal the output is the local attention.
    for (int i = lane; i < nq * (D / 8); i += 64) {
      const int q = i / (D / 8), c = i % (D / 8);
      const int t = q_first + q;
      *(uint4*)(p.out + b * p.out_sb + (int64_t)t * p.out_st + h * p.out_sh + c * 8) =
          *(const uint4*)(p.local + (((size_t)b * p.T + t) * p.H + h) * D + c * 8);
    }
  }

  // ---- union of the selected sets (ascending fine id) and per-wave masks
  for (int i = tid; i < kBitWords; i += kGroupThreads) sm.u.setup.bits[i] = 0;
  for (int i = tid; i < kMaxUnion / 4; i += kGroupThreads) sm.mask[i] = 0;
  // PERQ: this lane's query bitmask (rows li >= nq select nothing).
  const uint32_t* qbits = nullptr;
  if constexpr (PERQ) {
    for (int i = tid; i < kGroupWaves * kBitWords; i += kGroupThreads)
      (&sm.u.setup.wbits[0][0])[i] = 0u;
    if (reads)
      qbits = p.qsel + ((size_t)(b * p.T + q_first + min(li, nq - 1)) * p.H + h) * p.qsel_words;
  } else if (reads) {
    const int32_t* sel = p.sel_pool + ((size_t)slot * BH + bh) * p.sel_cap;
    for (int m = lane; m < M; m += 64) sm.ids[w][m] = sel[m];
  }
  __syncthreads();
  if constexpr (PERQ) {
    if (reads) {
      const int words = (p.first_epoch + erel + 31) >> 5;
      for (int i = 0; i < words; ++i) {
        uint32_t v = (lane < 32 && li < nq) ? qbits[i] : 0u;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) v |= __shfl_xor(v, off, 64);
        if (lane == 0) {
          sm.u.setup.wbits[w][i] = v;
          atomicOr(&sm.u.setup.bits[i], v);
        }
      }
    }
  } else if (reads) {
    for (int m = lane; m < M; m += 64) {
      const int id = sm.ids[w][m];
      atomicOr(&sm.u.setup.bits[id >> 5], 1u << (id & 31));
    }
  }
  __syncthreads();
  if (w == 0) {
    constexpr int WPL = kBitWords / 64;
    int cnt[WPL], total = 0;
#pragma unroll
    for (int i = 0; i < WPL; ++i) { cnt[i] = __popc(sm.u.setup.bits[lane * WPL + i]); total += cnt[i]; }
    int incl = total;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off, 64);
      if (lane >= off) incl += v;
    }
    int run = incl - total;
#pragma unroll
    for (int i = 0; i < WPL; ++i) { sm.u.setup.pre[lane * WPL + i] = run; run += cnt[i]; }
    if (lane == 63) sm.n_union = incl;
  }
  __syncthreads();
  for (int i = tid; i < kBitWords; i += kGroupThreads) {
    uint32_t bits = sm.u.setup.bits[i];
    int r = sm.u.setup.pre[i];
    while (bits) {
      const int bit = __ffs(bits) - 1;
      sm.uni[r] = i * 32 + bit;
      if constexpr (PERQ) {
        uint32_t byte = 0;
#pragma unroll
        for (int v = 0; v < kGroupWaves; ++v) byte |= ((sm.u.setup.wbits[v][i] >> bit) & 1u) << v;
        atomicOr(&sm.mask[r >> 2], byte << ((r & 3) * 8));
      }
      ++r;
      bits &= bits - 1;
    }
  }
  if (!PERQ && reads)
    for (int m = lane; m < M; m += 64) {
      const int id = sm.ids[w][m];
      const uint32_t word = sm.u.setup.bits[id >> 5];
      const int rank = sm.u.setup.pre[id >> 5] + __popc(word & ((1u << (id & 31)) - 1u));
      atomicOr(&sm.mask[rank >> 2], 1u << ((rank & 3) * 8 + w));
    }
  __syncthreads();
  const int U = sm.n_union;

  // ---- h of this wave's queries in the MFMA A layout: lane (li, hl) holds
  // row q = li, channels d = 16 kk + 8 hl + j (packed bf16).
  if (reads) {
    const int q = li < nq ? li : nq - 1;
    const bf16_t* rq = p.rq.p + b * p.rq.sb + (int64_t)(q_first + q) * p.rq.st + h * p.rq.sh;
    float x[KK][8];
    float mx = -__builtin_inff();
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      unpack8f(*(const uint4*)(rq + 16 * kk + 8 * hl), x[kk]);
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, x[kk][j]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sum = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) { x[kk][j] = __expf(x[kk][j] - mx); sum += x[kk][j]; }
    sum += __shfl_xor(sum, 32, 64);
    const float inv_valid = li < nq ? 1.0f : 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      uint32_t wv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wv[j] = pack_bf16x2(x[kk][2 * j] / sum * inv_valid, x[kk][2 * j + 1] / sum * inv_valid);
      *(uint4*)&sm.hq[w][li][16 * kk + 8 * hl] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    }
  }

  // ---- stream the union
  const bf16_t* bank = p.bank + (size_t)bh * p.fine_cap * D * D;
  const bf16_t* pw_base = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
  const bf16_t* psw_base = p.psw_pool ? p.psw_pool + ((size_t)erel * BH + bh) * 8 * D : nullptr;
  const bf16_t* sw_base = p.sw + (size_t)bh * p.fine_cap * D;
  auto active = [&](int u) __attribute__((always_inline)) { return reads && ((sm.mask[u >> 2] >> ((u & 3) * 8 + w)) & 1u); };
  // C^T rows of union entry u: thread tid moves uint4 chunks tid + i * 512,
  // i < CPT, into one of two named register sets (X = a or b).
  static_assert(CPT == 1 || CPT == 4, "head width 64 or 128");
#define TAO_C_CHUNK(i_) (bank + (size_t)cid * D * D + (size_t)(tid + (i_) * kGroupThreads) * 8)
#define TAO_LOAD_C(u, X)                                                 \
  do {                                                                   \
    const int cid = sm.uni[(u)];                                         \
    X##0 = *(const uint4*)TAO_C_CHUNK(0);                                \
    if constexpr (CPT == 4) {                                            \
      X##1 = *(const uint4*)TAO_C_CHUNK(1);                              \
      X##2 = *(const uint4*)TAO_C_CHUNK(2);                              \
      X##3 = *(const uint4*)TAO_C_CHUNK(3);                              \
    }                                                                    \
  } while (0)
#define TAO_C_SLOT(buf, i_)                                              \
  (*(uint4*)&sm.u.c[(buf)][(tid + (i_) * kGroupThreads) / CPR]           \
                  [((tid + (i_) * kGroupThreads) % CPR) * 8])
#define TAO_STORE_C(buf, X)                                              \
  do {                                                                   \
    TAO_C_SLOT(buf, 0) = X##0;                                           \
    if constexpr (CPT == 4) {                                            \
      TAO_C_SLOT(buf, 1) = X##1;                                         \
      TAO_C_SLOT(buf, 2) = X##2;                                         \
      TAO_C_SLOT(buf, 3) = X##3;                                         \
    }                                                                    \
  } while (0)
  // pw / sw rows of fine id for this wave: lane l < D / 2 moves 4 bytes of each.
  auto load_w = [&](int u, uint32_t& pwv, uint32_t& swv) __attribute__((always_inline)) {
    const int id = sm.uni[u];
    const bf16_t* pw = pw_base + (size_t)(id / p.group) * D;
    const bf16_t* sw = id < sw_split ? sw_base + (size_t)id * D : psw_base + (size_t)(id - sw_split) * D;
    if (lane < D / 2) {
      pwv = *(const uint32_t*)(pw + 2 * lane);
      swv = *(const uint32_t*)(sw + 2 * lane);
    }
  };
  auto store_w = [&](int buf, uint32_t pwv, uint32_t swv) __attribute__((always_inline)) {
    if (lane < D / 2) {
      *(uint32_t*)&sm.pwsw[w][buf][0][2 * lane] = pwv;
      *(uint32_t*)&sm.pwsw[w][buf][1][2 * lane] = swv;
    }
  };

  floatx16 acc[ET];
#pragma unroll
  for (int t = 0; t < ET; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
  floatx16 acc_den;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc_den[i] = 0.0f;
  // Pipeline: while fine u is consumed from LDS buffer u & 1, fine u + 1
  // waits in one register set (stored to LDS at the end of the iteration)
  // and fine u + 2's loads are in flight in the other, so each global load
  // has a whole iteration to arrive.
  uint4 a0, a1, a2, a3, b0, b1, b2, b3;
  uint32_t pwa = 0, swa = 0, pwb = 0, swb = 0;
  // Per wave: t = r(h * pw[page]) of the page last used, packed in the A
  // layout (consecutive union fines mostly share a page).
  uint4 tpk[KK];
  int cached_page = -1;
  const bf16x8 ones = as_bf16x8(make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u));
  // PERQ: the lane's bitmask word of the current fine (ids ascend).
  int qword_at = -1;
  uint32_t qword = 0u;
  auto consume = [&](int u) __attribute__((always_inline)) {
    if (!active(u)) return;
    const int buf = u & 1;
    const int page = sm.uni[u] / p.group;
    uint32_t keep = 0xFFFFFFFFu;
    if constexpr (PERQ) {
      const int id = sm.uni[u];
      if ((id >> 5) != qword_at) {
        qword_at = id >> 5;
        qword = li < nq ? qbits[qword_at] : 0u;
      }
      keep = ((qword >> (id & 31)) & 1u) ? 0xFFFFFFFFu : 0u;
    }
    if (page != cached_page) {
      const bf16_t* pwr = sm.pwsw[w][buf][0];
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int d0 = 16 * kk + 8 * hl;
        float hv[8], pv[8];
        unpack8f(*(const uint4*)&sm.hq[w][li][d0], hv);
        unpack8f(*(const uint4*)(pwr + d0), pv);
        uint32_t t1[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          t1[j] = pack_bf16x2(hv[2 * j] * pv[2 * j], hv[2 * j + 1] * pv[2 * j + 1]);
        tpk[kk] = make_uint4(t1[0], t1[1], t1[2], t1[3]);
      }
      cached_page = page;
    }
    const bf16_t* swr = sm.pwsw[w][buf][1];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int d0 = 16 * kk + 8 * hl;
      float tv[8], sv[8];
      unpack8f(tpk[kk], tv);
      unpack8f(*(const uint4*)(swr + d0), sv);
      uint32_t ch[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ch[j] = pack_bf16x2(tv[2 * j] * sv[2 * j], tv[2 * j + 1] * sv[2 * j + 1]) & keep;
      const bf16x8 a = as_bf16x8(make_uint4(ch[0], ch[1], ch[2], ch[3]));
#pragma unroll
      for (int t = 0; t < ET; ++t) {
        const bf16x8 bq = as_bf16x8(*(const uint4*)&sm.u.c[buf][32 * t + li][d0]);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bq, acc[t], 0, 0, 0);
      }
      // den: the same A against a column of ones.
      acc_den = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, ones, acc_den, 0, 0, 0);
    }
  };
  if (U > 0) {
    TAO_LOAD_C(0, a);
    if (active(0)) load_w(0, pwa, swa);
    TAO_STORE_C(0, a);
    if (active(0)) store_w(0, pwa, swa);
  }
  if (U > 1) {
    TAO_LOAD_C(1, b);
    if (active(1)) load_w(1, pwb, swb);
  }
  __syncthreads();
  // Even u: fine u + 2 -> set a, fine u + 1 (set b) -> LDS; odd u: the reverse.
  for (int u = 0; u < U; u += 2) {
    if (u + 2 < U) {
      TAO_LOAD_C(u + 2, a);
      if (active(u + 2)) load_w(u + 2, pwa, swa);
    }
    consume(u);
    if (u + 1 < U) {
      TAO_STORE_C(1, b);
      if (active(u + 1)) store_w(1, pwb, swb);
    }
    __syncthreads();
    if (u + 1 >= U) break;
    if (u + 3 < U) {
      TAO_LOAD_C(u + 3, b);
      if (active(u + 3)) load_w(u + 3, pwb, swb);
    }
    consume(u + 1);
    if (u + 2 < U) {
      TAO_STORE_C(0, a);
      if (active(u + 2)) store_w(0, pwa, swa);
    }
    __syncthreads();
  }

#undef TAO_LOAD_C
#undef TAO_STORE_C
#undef TAO_C_SLOT
#undef TAO_C_CHUNK
  // ---- epilogue: fine = r(r(num) / r(den)), the coarse read, the fusion.
  if (!reads) return;
  const bool coarse_on = COARSE && cpages >= 1;
  const bf16_t* gc =
      coarse_on ? p.coarse_pool + ((size_t)(cpages - p.coarse_first) * BH + bh) * D * D : nullptr;
  // One e-tile of the accumulator (called with constant t, so acc stays in
  // registers).
  auto emit = [&](const floatx16& av, int t) __attribute__((always_inline)) {
    const int e = 32 * t + li;
    float ae[3], be[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      ae[i] = load_param(p.fa, p.f_dtype, h * p.fa_s[0] + e * p.fa_s[1] + i * p.fa_s[2]);
      be[i] = load_param(p.fb, p.f_dtype, h * p.fb_s[0] + e * p.fb_s[1] + i * p.fb_s[2]);
    }
    // coarse[q][e] = h_q . G^T[e]: A = the wave's h rows, B = G^T rows of
    // this e-tile (k = d contiguous).
    floatx16 cacc;
#pragma unroll
    for (int i = 0; i < 16; ++i) cacc[i] = 0.0f;
    if constexpr (COARSE) {
      if (coarse_on) {
        uint4 gb[KK];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          gb[kk] = *(const uint4*)(gc + (size_t)e * D + 16 * kk + 8 * hl);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              as_bf16x8(*(const uint4*)&sm.hq[w][li][16 * kk + 8 * hl]), as_bf16x8(gb[kk]),
              cacc, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int q = 8 * (i / 4) + 4 * hl + (i % 4);
      if (q < nq) {
        const int tq = q_first + q;
        const float fine = rbf(rbf(av[i]) * __builtin_amdgcn_rcpf(rbf(acc_den[i])));
        const size_t row = ((size_t)b * p.T + tq) * p.H + h;
        if (p.save_fine) {
          p.save_fine[row * D + e] = f2bf(fine);
          p.save_coarse[row * D + e] = f2bf(rbf(cacc[i]));
          if (e == 0) p.save_den[row] = rbf(acc_den[i]);
        }
        const float local = bf2f(p.local[(((size_t)b * p.T + tq) * p.H + h) * D + e]);
        const float x = bf2f(p.rq.p[b * p.rq.sb + (int64_t)tq * p.rq.st + h * p.rq.sh + e]);
        p.out[b * p.out_sb + (int64_t)tq * p.out_st + h * p.out_sh + e] =
            fuse_element(x, local, rbf(cacc[i]), fine, ae, be, p.gain, coarse_on ? 1 : 0, 1);
      }
    }
  };
  static_assert(ET == 2 || ET == 4, "head width 64 or 128");
  emit(acc[0], 0);
  emit(acc[1], 1);
  if constexpr (ET == 4) {
    emit(acc[2], 2);
    emit(acc[3], 3);
  }
}

}  // namespace

hipError_t launch_pages(const PagesParams& p, int head_dim, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  if (p.group != 8) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(p.count * p.B * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(pages_kernel<128>, grid, dim3(kThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(pages_kernel<64>, grid, dim3(kThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_epochs(const EpochParams& p, int head_dim, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  if (p.group != 8) return hipErrorInvalidValue;
  const int last_pages = (p.first_epoch + p.count - 1) / p.group + 1;
  if (last_pages > 64 * 32 || last_pages > p.pool_pcap) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(p.count * p.B * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(epochs_kernel<128>, grid, dim3(kThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(epochs_kernel<64>, grid, dim3(kThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_read_tiles(const ReadTilesParams& p, int head_dim, hipStream_t s) {
  if (p.n_tiles <= 0) return hipSuccess;
  if (p.fine_cap > kMaxFineIds) return hipErrorInvalidValue;
  const int groups = (p.n_tiles + kGroupWaves - 1) / kGroupWaves;
  const dim3 grid((unsigned)(groups * p.B * p.H));
  const bool coarse = p.coarse_pool != nullptr;
  const bool perq = p.qsel != nullptr;
  if (perq && (p.qsel_words < 1 || p.qsel_words > kBitWords)) return hipErrorInvalidValue;
#define TAO_READ_LAUNCH(D_, C_, Q_)                                                           \
  hipLaunchKernelGGL((read_groups_kernel<D_, C_, Q_>), grid, dim3(kGroupThreads), 0, s, p)
  if (head_dim != 128 && head_dim != 64) return hipErrorInvalidValue;
  if (head_dim == 128) {
    if (perq) {
      if (coarse) TAO_READ_LAUNCH(128, true, true); else TAO_READ_LAUNCH(128, false, true);
    } else {
      if (coarse) TAO_READ_LAUNCH(128, true, false); else TAO_READ_LAUNCH(128, false, false);
    }
  } else {
    if (perq) {
      if (coarse) TAO_READ_LAUNCH(64, true, true); else TAO_READ_LAUNCH(64, false, true);
    } else {
      if (coarse) TAO_READ_LAUNCH(64, true, false); else TAO_READ_LAUNCH(64, false, false);
    }
  }
#undef TAO_READ_LAUNCH
  return hipGetLastError();
}

}  // namespace tao
