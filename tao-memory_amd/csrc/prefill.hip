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
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
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
  const float pz =
      p.fine_mass ? mass_page_z(p.fine_mass + ((size_t)bh * p.fine_cap + g * p.group) * D + d, 8, D)
                  : group_logsumexp(zv, 8);
  p.page_z[((size_t)bh * p.page_cap + g) * D + d] = f2bf(pz);
  for (int i = 0; i < 8; ++i)
    p.fine_sw[((size_t)bh * p.fine_cap + g * p.group + i) * D + d] = f2bf(exp_bf(rbf(zv[i] - pz)));
}

// One workgroup per (epoch, batch, head): the pending page summary with one
// thread per channel, then the page weights, a segment of lanes (one lane
// per page) per channel.
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
    const float pz =
        p.fine_mass
            ? mass_page_z(p.fine_mass + ((size_t)bh * p.fine_cap + K * p.group) * D + tid, pend, D)
            : group_logsumexp(zv, pend);
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
  auto desc = [&](int pg, int d) __attribute__((always_inline)) {
    return pg == K ? pend_pz[d] : bf2f(pzg[(size_t)pg * D + d]);
  };
  if (P <= 64) {
    // Segments of W = pow2 >= P lanes, one channel each (64 / W channels per
    // pass of a wave). The lanes past P hold zeros, so the segment's xor fold
    // adds exactly what wave_sum_fold adds over 64 lanes.
    int W = 1;
    while (W < P) W <<= 1;
    const int per = 64 / W, pg = lane % W;
    for (int d0 = wave * per; d0 < D; d0 += (kThreads / 64) * per) {
      const int d = d0 + lane / W;
      const float x = pg < P ? desc(pg, d) : -__builtin_inff();
      float m = x;
      for (int off = W / 2; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
      const float e = pg < P ? exp_cr(x - m) : 0.0f;
      float total = e;
      for (int off = W / 2; off >= 1; off >>= 1) total += __shfl_xor(total, off, 64);
      if (pg < P) {
        const bf16_t w = f2bf(e / total);
        pw[(size_t)pg * D + d] = w;
        if (last) state_pw[(size_t)pg * D + d] = w;
      }
    }
    return;
  }
  for (int d = wave; d < D; d += kThreads / 64) {
    page_weights_wave(
        lane, P, [&](int pg) { return desc(pg, d); },
        [&](int pg, bf16_t w) {
          pw[(size_t)pg * D + d] = w;
          if (last) state_pw[(size_t)pg * D + d] = w;
        });
  }
}

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
    bf16_t c[2][D][D + 8];        // staged weighted C^T, rows padded by 16 bytes
  } u;
  bf16_t wr[2][D];                     // per buffer: the staged fine's weights r(pw * sw)
  float ez[2][D];                      // feature writers: exp(z) of the staged fine
  int ids[kGroupWaves][kMaxM];
  int uni[kMaxUnion];
  uint32_t mask[kMaxUnion / 4];        // byte u: bit w set if wave w selected uni[u]
  int n_union;
  int erels[kGroupWaves];              // each wave's tile epoch, -1 without a read
};

TAO_DEV void unpack8f(const uint4& u, float out[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

// Eight bf16 weights r(pw * sw) of one 16-byte slice, packed.
TAO_DEV uint4 slice_weights(const uint4& pw, const uint4& sw) {
  float a[8], b[8];
  unpack8f(pw, a);
  unpack8f(sw, b);
  return make_uint4(pack_bf16x2(a[0] * b[0], a[1] * b[1]), pack_bf16x2(a[2] * b[2], a[3] * b[3]),
                    pack_bf16x2(a[4] * b[4], a[5] * b[5]), pack_bf16x2(a[6] * b[6], a[7] * b[7]));
}

// One 16-byte slice of C^T scaled by the slice's weights, rounded to bf16.
TAO_DEV uint4 scale_slice(const uint4& c, const uint4& wr) {
  float a[8], b[8];
  unpack8f(c, a);
  unpack8f(wr, b);
  return make_uint4(pack_bf16x2(a[0] * b[0], a[1] * b[1]), pack_bf16x2(a[2] * b[2], a[3] * b[3]),
                    pack_bf16x2(a[4] * b[4], a[5] * b[5]), pack_bf16x2(a[6] * b[6], a[7] * b[7]));
}

// Turn-group read: one 512-thread workgroup per (8 consecutive read tiles,
// batch, head); wave w owns tile w (<= 32 queries sharing one route, its
// own seal epoch and segment-weight source). The read of a fine is linear in
// its channel weights, num[q][e] = sum_d h_q[d] w[d] C^T[e][d] with
// w = r(pw[page] * sw[fine]) shared by every tile of one seal epoch, so the
// workgroup stages each fine's C^T already weighted (r(C^T * w), padded LDS,
// double-buffered, the next fine's rows and weight slices in flight in
// registers) and every tile's A operand is its queries' h, which stays in
// registers for the whole kernel: a selecting wave runs 4 x 8
// v_mfma_f32_32x32x16_bf16 into its 32 x D accumulator plus 8 against the
// weights for den[q] = sum over its fines of h_q . w, with no per-fine VALU.
// The workgroup takes one pass per distinct epoch among its tiles (a group
// straddles at most a seal): each pass streams the union of its tiles'
// selected sets. fine = r(r(num) / r(den)), then the fusion epilogue. The
// reference rounds h * pw and then the product with sw to bf16 before its
// fp32 sums (selected_read.py:31, 48); here the product of the two weights
// is rounded and folded into C, which moves the read within its bf16
// tolerance. With the coarse value branch (COARSE), each e-tile of a tile
// whose chunk has completed pages also runs 8 MFMAs of the wave's h against
// the folded coarse matrix of its page count (coarse.hip) before the fusion.
//
// PERQ (the full-sequence read, every query routed by itself): selections
// are per-query bitmasks (route_queries_kernel). The union and the per-wave
// masks come from the OR of the wave's bitmasks, and each A row is zeroed
// unless its own query selected the fine, so a wave's 32 queries still share
// every staged C^T and MFMA; the numerator and denominator of a query sum
// exactly its selected fines (selected_read.py:156-173).
template <int D, bool COARSE, bool PERQ, bool FEAT>
__global__ __launch_bounds__(kGroupThreads) void read_groups_kernel(ReadTilesParams p) {
  static_assert(!FEAT || PERQ, "the group read's mixture serves per-query reads");
  constexpr int KK = D / 16, ET = D / 32, CPR = D / 8;   // k-steps, e-tiles, uint4 per row
  constexpr int CPT = D * CPR / kGroupThreads;           // C^T uint4 per thread
  static_assert(CPT == 1 || CPT == 4, "head width 64 or 128");
  static_assert(kGroupThreads % CPR == 0, "a thread's C^T chunks share one column slice");
  __shared__ GroupSmem<D> sm;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  // Tiles in reverse plan order: the latest tiles read the most fines, so
  // they start first and the light early tiles fill the end of the launch.
  const int grp = (p.n_tiles + kGroupWaves - 1) / kGroupWaves - 1 - (int)blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const int t0 = grp * kGroupWaves;
  const int nt = min(kGroupWaves, p.n_tiles - t0);
  const int cc = tid % CPR;                              // this thread's column slice

  // This wave's tile.
  int q_first = 0, nq = 0, slot = 0, M = 0, erel = 0, fine_on = 0, cpages = 0;
  if (w < nt) {
    const int64_t* desc = p.tiles + 8 * (t0 + w);
    q_first = (int)desc[0]; nq = (int)desc[1]; slot = (int)desc[2]; M = (int)desc[3];
    erel = (int)desc[4]; fine_on = (int)desc[6];
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
  if (lane == 0) sm.erels[w] = reads ? erel : -1;

  // ---- h of this wave's queries in the MFMA A layout, kept in registers:
  // lane (li, hl) holds row q = li, channels d = 16 kk + 8 hl + j (packed
  // bf16); rows past the tile are zero.
  uint4 hA[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) hA[kk] = make_uint4(0u, 0u, 0u, 0u);
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
    // One reciprocal per row: h only shapes the read (within its tolerance),
    // never a route.
    const float inv = li < nq ? __builtin_amdgcn_rcpf(sum) : 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      uint32_t wv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wv[j] = pack_bf16x2(x[kk][2 * j] * inv, x[kk][2 * j + 1] * inv);
      hA[kk] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    }
  }
  // PERQ: this lane's query bitmask (rows li >= nq select nothing).
  const uint32_t* qbits = nullptr;
  if constexpr (PERQ) {
    if (reads)
      qbits = p.qsel + ((size_t)(b * p.T + q_first + min(li, nq - 1)) * p.H + h) * p.qsel_words;
  }

  // Feature writers: the query's mixture normaliser, the sum over its
  // selected fines (ascending id) of mass = sum_d h[d] exp(z[d]) in fp32,
  // the same order as each fine's mass in the read.
  auto h_of = [&](int kk, float hv[8]) __attribute__((always_inline)) { unpack8f(hA[kk], hv); };
  float tot = 0.0f;
  if constexpr (FEAT) {
    if (reads && li < nq) {
      const int words = (p.first_epoch + erel + 31) >> 5;
      const bf16_t* zb = p.fine_z + (size_t)bh * p.fine_cap * D;
      for (int i = 0; i < words; ++i) {
        uint32_t bits = qbits[i];
        while (bits) {
          const int f = i * 32 + __ffs(bits) - 1;
          bits &= bits - 1;
          float part = 0.0f;
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) {
            float hv[8], zf[8];
            h_of(kk, hv);
            unpack8f(*(const uint4*)(zb + (size_t)f * D + 16 * kk + 8 * hl), zf);
#pragma unroll
            for (int j = 0; j < 8; ++j) part += hv[j] * expf(zf[j]);
          }
          part += __shfl_xor(part, 32, 64);
          tot += part;
        }
      }
    }
  }

  floatx16 acc[ET];
#pragma unroll
  for (int t = 0; t < ET; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
  floatx16 acc_den;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc_den[i] = 0.0f;

  const bf16_t* bank = p.bank + (size_t)bh * p.fine_cap * D * D;
  const bf16_t* sw_base = p.sw + (size_t)bh * p.fine_cap * D;
  __syncthreads();   // sm.erels

  // ---- one pass per distinct epoch of the group's reading tiles, ascending
  for (int pass_erel = -1;;) {
    int next = 0x7FFFFFFF;
#pragma unroll
    for (int v = 0; v < kGroupWaves; ++v) {
      const int e = sm.erels[v];
      if (e > pass_erel && e < next) next = e;
    }
    if (next == 0x7FFFFFFF) break;
    pass_erel = next;
    const bool in_pass = reads && erel == pass_erel;
    // The pass's page weights (its epoch pool) and segment-weight source:
    // fines below the epoch's completed pages read the state's weights, the
    // pending page's fines the epoch's pool rows.
    const int pass_epoch = p.first_epoch + pass_erel;
    const int sw_split = (pass_epoch / p.group) * p.group;
    const bf16_t* pw_base = p.pw_pool + ((size_t)pass_erel * BH + bh) * p.pool_pcap * D;
    const bf16_t* psw_base =
        p.psw_pool ? p.psw_pool + ((size_t)pass_erel * BH + bh) * 8 * D : nullptr;

    // ---- union of the pass's selected sets (ascending fine id), per-wave masks
    for (int i = tid; i < kBitWords; i += kGroupThreads) sm.u.setup.bits[i] = 0;
    for (int i = tid; i < kMaxUnion / 4; i += kGroupThreads) sm.mask[i] = 0;
    if constexpr (PERQ) {
      for (int i = tid; i < kGroupWaves * kBitWords; i += kGroupThreads)
        (&sm.u.setup.wbits[0][0])[i] = 0u;
    } else if (in_pass) {
      const int32_t* sel = p.sel_pool + ((size_t)slot * BH + bh) * p.sel_cap;
      for (int m = lane; m < M; m += 64) sm.ids[w][m] = sel[m];
    }
    __syncthreads();
    if constexpr (PERQ) {
      if (in_pass) {
        const int words = (pass_epoch + 31) >> 5;
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
    } else if (in_pass) {
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
      for (int i = 0; i < WPL; ++i) {
        cnt[i] = __popc(sm.u.setup.bits[lane * WPL + i]);
        total += cnt[i];
      }
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
          for (int v = 0; v < kGroupWaves; ++v)
            byte |= ((sm.u.setup.wbits[v][i] >> bit) & 1u) << v;
          atomicOr(&sm.mask[r >> 2], byte << ((r & 3) * 8));
        }
        ++r;
        bits &= bits - 1;
      }
    }
    if (!PERQ && in_pass)
      for (int m = lane; m < M; m += 64) {
        const int id = sm.ids[w][m];
        const uint32_t word = sm.u.setup.bits[id >> 5];
        const int rank = sm.u.setup.pre[id >> 5] + __popc(word & ((1u << (id & 31)) - 1u));
        atomicOr(&sm.mask[rank >> 2], 1u << ((rank & 3) * 8 + w));
      }
    __syncthreads();
    const int U = sm.n_union;

    // ---- stream the union. Thread tid moves C^T chunks tid + i * 512 (i <
    // CPT, all in column slice cc) and that slice of the fine's pw and sw
    // rows through one of two named register sets (X = a or b).
    auto active = [&](int u) __attribute__((always_inline)) {
      return in_pass && ((sm.mask[u >> 2] >> ((u & 3) * 8 + w)) & 1u);
    };
#define TAO_C_CHUNK(i_) (bank + (size_t)cid * D * D + (size_t)(tid + (i_) * kGroupThreads) * 8)
#define TAO_LOAD_C(u, X)                                                           \
  do {                                                                             \
    const int cid = sm.uni[(u)];                                                   \
    if constexpr (FEAT) {                                                          \
      X##p = *(const uint4*)(p.fine_z + ((size_t)bh * p.fine_cap + cid) * D + cc * 8); \
    } else {                                                                       \
      const bf16_t* swr_ = cid < sw_split ? sw_base + (size_t)cid * D              \
                                          : psw_base + (size_t)(cid - sw_split) * D; \
      X##p = *(const uint4*)(pw_base + (size_t)(cid / p.group) * D + cc * 8);      \
      X##s = *(const uint4*)(swr_ + cc * 8);                                       \
    }                                                                              \
    X##0 = *(const uint4*)TAO_C_CHUNK(0);                                          \
    if constexpr (CPT == 4) {                                                      \
      X##1 = *(const uint4*)TAO_C_CHUNK(1);                                        \
      X##2 = *(const uint4*)TAO_C_CHUNK(2);                                        \
      X##3 = *(const uint4*)TAO_C_CHUNK(3);                                        \
    }                                                                              \
  } while (0)
#define TAO_C_SLOT(buf, i_)                                              \
  (*(uint4*)&sm.u.c[(buf)][(tid + (i_) * kGroupThreads) / CPR][cc * 8])
#define TAO_STORE_C(buf, X)                                              \
  do {                                                                   \
    if constexpr (FEAT) {                                                \
      if (tid < CPR) {                                                   \
        float zf_[8];                                                    \
        unpack8f(X##p, zf_);                                             \
        _Pragma("unroll") for (int j_ = 0; j_ < 8; ++j_)                 \
          sm.ez[(buf)][cc * 8 + j_] = expf(zf_[j_]);                     \
      }                                                                  \
      TAO_C_SLOT(buf, 0) = X##0;                                         \
      if constexpr (CPT == 4) {                                          \
        TAO_C_SLOT(buf, 1) = X##1;                                       \
        TAO_C_SLOT(buf, 2) = X##2;                                       \
        TAO_C_SLOT(buf, 3) = X##3;                                       \
      }                                                                  \
      break;                                                             \
    }                                                                    \
    const uint4 wr_ = slice_weights(X##p, X##s);                         \
    if (tid < CPR) *(uint4*)&sm.wr[(buf)][cc * 8] = wr_;                 \
    TAO_C_SLOT(buf, 0) = scale_slice(X##0, wr_);                         \
    if constexpr (CPT == 4) {                                            \
      TAO_C_SLOT(buf, 1) = scale_slice(X##1, wr_);                       \
      TAO_C_SLOT(buf, 2) = scale_slice(X##2, wr_);                       \
      TAO_C_SLOT(buf, 3) = scale_slice(X##3, wr_);                       \
    }                                                                    \
  } while (0)

    // PERQ: the lane's bitmask word of the current fine (ids ascend).
    int qword_at = -1;
    uint32_t qword = 0u;
    auto consume = [&](int u) __attribute__((always_inline)) {
      if (!active(u)) return;
      const int buf = u & 1;
      uint32_t keep = 0xFFFFFFFFu;
      if constexpr (PERQ) {
        const int id = sm.uni[u];
        if ((id >> 5) != qword_at) {
          qword_at = id >> 5;
          qword = li < nq ? qbits[qword_at] : 0u;
        }
        keep = ((qword >> (id & 31)) & 1u) ? 0xFFFFFFFFu : 0u;
      }
      if constexpr (FEAT) {
        // coef = r(mix * h) with mix = mass / tot of this fine, rows of
        // queries that did not select it zero; no denominator.
        float part = 0.0f;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          float hv[8];
          h_of(kk, hv);
          const float* ez = &sm.ez[buf][16 * kk + 8 * hl];
#pragma unroll
          for (int j = 0; j < 8; ++j) part += hv[j] * ez[j];
        }
        part += __shfl_xor(part, 32, 64);
        const float mix = keep ? part / tot : 0.0f;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          const int d0 = 16 * kk + 8 * hl;
          float hv[8];
          h_of(kk, hv);
          const bf16x8 a = as_bf16x8(make_uint4(
              pack_bf16x2(mix * hv[0], mix * hv[1]), pack_bf16x2(mix * hv[2], mix * hv[3]),
              pack_bf16x2(mix * hv[4], mix * hv[5]), pack_bf16x2(mix * hv[6], mix * hv[7])));
#pragma unroll
          for (int t = 0; t < ET; ++t) {
            const bf16x8 bq = as_bf16x8(*(const uint4*)&sm.u.c[buf][32 * t + li][d0]);
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bq, acc[t], 0, 0, 0);
          }
        }
        return;
      }
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int d0 = 16 * kk + 8 * hl;
        uint4 av = hA[kk];
        if constexpr (PERQ) { av.x &= keep; av.y &= keep; av.z &= keep; av.w &= keep; }
        const bf16x8 a = as_bf16x8(av);
#pragma unroll
        for (int t = 0; t < ET; ++t) {
          const bf16x8 bq = as_bf16x8(*(const uint4*)&sm.u.c[buf][32 * t + li][d0]);
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bq, acc[t], 0, 0, 0);
        }
        // den: the same A against the fine's weights in every column.
        const bf16x8 wq = as_bf16x8(*(const uint4*)&sm.wr[buf][d0]);
        acc_den = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, wq, acc_den, 0, 0, 0);
      }
    };
    uint4 a0, a1, a2, a3, ap, as, b0, b1, b2, b3, bp, bs;
    if (U > 0) {
      TAO_LOAD_C(0, a);
      TAO_STORE_C(0, a);
    }
    if (U > 1) TAO_LOAD_C(1, b);
    __syncthreads();
    // Even u: fine u + 2 -> set a, fine u + 1 (set b) -> LDS; odd u: the reverse.
    for (int u = 0; u < U; u += 2) {
      if (u + 2 < U) TAO_LOAD_C(u + 2, a);
      consume(u);
      if (u + 1 < U) TAO_STORE_C(1, b);
      __syncthreads();
      if (u + 1 >= U) break;
      if (u + 3 < U) TAO_LOAD_C(u + 3, b);
      consume(u + 1);
      if (u + 2 < U) TAO_STORE_C(0, a);
      __syncthreads();
    }
#undef TAO_LOAD_C
#undef TAO_STORE_C
#undef TAO_C_SLOT
#undef TAO_C_CHUNK
    __syncthreads();   // the next pass's setup reuses the staging buffers
  }

  // ---- epilogue: fine = r(r(num) / r(den)), the coarse read, the fusion.
  if (!reads) return;
  const bool coarse_on = COARSE && cpages >= 1;
  const bf16_t* gc = coarse_on && !FEAT
                         ? p.coarse_pool + ((size_t)(cpages - p.coarse_first) * BH + bh) * D * D
                         : nullptr;
  // Feature writers with page values: the mixture of the chunk's completed
  // pages (tao_stream.py:301-305, 609-615), mass_p = sum_d h[d] exp(page_z[p][d]).
  const bf16_t* pzb = FEAT && coarse_on ? p.page_z + (size_t)bh * p.page_cap * D : nullptr;
  const bf16_t* pcb = FEAT && coarse_on ? p.page_c + (size_t)bh * p.page_cap * D * D : nullptr;
  auto page_mass = [&](int pg) __attribute__((always_inline)) {
    float part = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      float hv[8], zf[8];
      h_of(kk, hv);
      unpack8f(*(const uint4*)(pzb + (size_t)pg * D + 16 * kk + 8 * hl), zf);
#pragma unroll
      for (int j = 0; j < 8; ++j) part += hv[j] * expf(zf[j]);
    }
    return part + __shfl_xor(part, 32, 64);
  };
  float totc = 0.0f;
  if constexpr (FEAT && COARSE) {
    if (coarse_on)
      for (int pg = 0; pg < cpages; ++pg) totc += page_mass(pg);
  }
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
    if constexpr (COARSE && FEAT) {
      if (coarse_on) {
        for (int pg = 0; pg < cpages; ++pg) {
          const float mix = page_mass(pg) / totc;
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) {
            float hv[8];
            h_of(kk, hv);
            const bf16x8 a = as_bf16x8(make_uint4(
                pack_bf16x2(mix * hv[0], mix * hv[1]), pack_bf16x2(mix * hv[2], mix * hv[3]),
                pack_bf16x2(mix * hv[4], mix * hv[5]), pack_bf16x2(mix * hv[6], mix * hv[7])));
            const uint4 gb = *(const uint4*)(pcb + ((size_t)pg * D + e) * D + 16 * kk + 8 * hl);
            cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, as_bf16x8(gb), cacc, 0, 0, 0);
          }
        }
      }
    } else if constexpr (COARSE) {
      if (coarse_on) {
        uint4 gb[KK];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          gb[kk] = *(const uint4*)(gc + (size_t)e * D + 16 * kk + 8 * hl);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(hA[kk]), as_bf16x8(gb[kk]),
                                                         cacc, 0, 0, 0);
      }
    }
    // Every operand of the 16 outputs first (rows past the tile clamped),
    // so the loads are in flight together rather than one round trip per
    // output behind the previous output's store.
    float lv[16], xv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int q = min(8 * (i / 4) + 4 * hl + (i % 4), nq - 1);
      const int tq = q_first + q;
      lv[i] = bf2f(p.local[(((size_t)b * p.T + tq) * p.H + h) * D + e]);
      xv[i] = bf2f(p.rq.p[b * p.rq.sb + (int64_t)tq * p.rq.st + h * p.rq.sh + e]);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int q = 8 * (i / 4) + 4 * hl + (i % 4);
      if (q < nq) {
        const int tq = q_first + q;
        const float fine =
            FEAT ? rbf(av[i]) : rbf(rbf(av[i]) * __builtin_amdgcn_rcpf(rbf(acc_den[i])));
        const size_t row = ((size_t)b * p.T + tq) * p.H + h;
        if (p.save_fine) {
          p.save_fine[row * D + e] = f2bf(fine);
          p.save_coarse[row * D + e] = f2bf(rbf(cacc[i]));
          // The mixture read has no denominator: 1 keeps the fusion
          // adjoint's d num = d fine / den exact.
          if (e == 0) p.save_den[row] = FEAT ? 1.0f : rbf(acc_den[i]);
        }
        p.out[b * p.out_sb + (int64_t)tq * p.out_st + h * p.out_sh + e] =
            fuse_element(xv[i], lv[i], rbf(cacc[i]), fine, ae, be, p.gain, coarse_on ? 1 : 0, 1);
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


// The fusion row phase of a turn-group read: lane (row r, unit c) fuses
// channels 8 c .. 8 c + 7 of query r of the wave's tile from the tile's fine
// and coarse values in LDS ([q][e], 16-byte units XOR-swizzled by the row),
// the local attention and the raw query, and stores the output. STAGED: the
// fusion parameters come from LDS, fpar[0][d][i] = a[h][d][i] and
// fpar[1][d][i] = b[h][d][i].
template <int D, bool COARSE, bool STAGED>
TAO_DEV void fuse_rows(const ReadTilesParams& p, const float (*fpar)[D * 3], const bf16_t* tile_f,
                       const bf16_t* tile_c, int lane, int b, int h, int q_first, int nq,
                       bool coarse_on) {
  constexpr int CPR = D / 8;
  auto unit_at = [&](int row, int unit) __attribute__((always_inline)) {
    return row * D + 8 * (unit ^ (row % CPR));
  };
  // Row phase: lane (row r, unit c) fuses channels 8 c .. 8 c + 7 of query r.
  constexpr int RPI = 64 / CPR;                 // rows per pass of the wave
  const int c = lane % CPR;
  float ae[8][3], be[8][3];
  if constexpr (STAGED) {
#pragma unroll
    for (int v = 0; v < 6; ++v) {
      const float4 av = *(const float4*)&fpar[0][24 * c + 4 * v];
      const float4 bv = *(const float4*)&fpar[1][24 * c + 4 * v];
      const float af[4] = {av.x, av.y, av.z, av.w}, bf[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ae[(4 * v + e) / 3][(4 * v + e) % 3] = af[e];
        be[(4 * v + e) / 3][(4 * v + e) % 3] = bf[e];
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        ae[j][i] = load_param(p.fa, p.f_dtype, h * p.fa_s[0] + (8 * c + j) * p.fa_s[1] + i * p.fa_s[2]);
        be[j][i] = load_param(p.fb, p.f_dtype, h * p.fb_s[0] + (8 * c + j) * p.fb_s[1] + i * p.fb_s[2]);
      }
  }
  // Without the coarse branch: the paired two-channel fusion on the rounded
  // parameters and the signed-zero coarse term.
  float ra[8][3], rb[8][3];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      ra[j][i] = rbf(ae[j][i]);
      rb[j][i] = rbf(be[j][i]);
    }
  const float ct0 = rbf(0.0f * rbf(p.gain * 0.0f));
  // Every pass's local and query rows are loaded first (rows past the tile
  // read its last row), so the passes do not wait on memory one by one
  // behind the previous pass's stores.
  constexpr int ITS = 32 / RPI;
  uint4 lus[ITS], xus[ITS];
#pragma unroll
  for (int it = 0; it < ITS; ++it) {
    const int tq = q_first + min(lane / CPR + RPI * it, nq - 1);
    lus[it] = *(const uint4*)(p.local + (((size_t)b * p.T + tq) * p.H + h) * D + 8 * c);
    xus[it] = *(const uint4*)(p.rq.p + b * p.rq.sb + (int64_t)tq * p.rq.st + h * p.rq.sh + 8 * c);
  }
#pragma unroll
  for (int it = 0; it < ITS; ++it) {
    const int r = lane / CPR + RPI * it;
    if (r >= nq) break;
    const int tq = q_first + r;
    const size_t row = ((size_t)b * p.T + tq) * p.H + h;
    const uint4 fu = *(const uint4*)&tile_f[unit_at(r, c)];
    uint4 cu = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (COARSE) {
      if (coarse_on) cu = *(const uint4*)&tile_c[unit_at(r, c)];
    }
    const uint4 lu = lus[it];
    const uint4 xu = xus[it];
    float fv[8], cv[8], lv[8], xv[8];
    unpack8f(fu, fv);
    unpack8f(cu, cv);
    unpack8f(lu, lv);
    unpack8f(xu, xv);
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (!COARSE) {
        o[j] = fuse_pair_local_fine(&xv[2 * j], &lv[2 * j], &fv[2 * j], &ra[2 * j], &rb[2 * j],
                                    p.gain, ct0);
      } else {
        const bf16_t lo = fuse_element(xv[2 * j], lv[2 * j], cv[2 * j], fv[2 * j], ae[2 * j],
                                       be[2 * j], p.gain, coarse_on ? 1 : 0, 1);
        const bf16_t hi = fuse_element(xv[2 * j + 1], lv[2 * j + 1], cv[2 * j + 1], fv[2 * j + 1],
                                       ae[2 * j + 1], be[2 * j + 1], p.gain, coarse_on ? 1 : 0, 1);
        o[j] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
               ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
      }
    }
    *(uint4*)(p.out + b * p.out_sb + (int64_t)tq * p.out_st + h * p.out_sh + 8 * c) =
        make_uint4(o[0], o[1], o[2], o[3]);
    if (p.save_fine) {
      *(uint4*)(p.save_fine + row * D + 8 * c) = fu;
      *(uint4*)(p.save_coarse + row * D + 8 * c) = cu;
    }
  }
}

// ---- Turn-route read with a ring of fines staged by direct loads into LDS.
//
// read_stream_kernel serves the prefill (turn routes; per-query routes take
// read_groups_kernel). It is read_groups_kernel's turn-group read with the
// staging replaced: each fine's C^T goes from HBM straight into one of
// kRing LDS slots (global_load_lds_dwordx4: lane i of a wave writes 16
// bytes at the slot's base + 16 i, so the lane picks which global chunk
// lands there; rows are stored with their 16-byte chunks XOR-swizzled by the
// row index, which keeps the B-operand reads free of bank conflicts). Fines
// go in pairs: fines u and u + 1 are read from two slots while u + 2 and
// u + 3 load into the other two, one barrier per pair. Wave 0 also moves a
// fine's pw and sw rows into LDS and turns them into the fine's weights
// w = r(pw * sw) before the barrier that publishes the fine. A selecting
// wave's A operand is r(h * w), and den[q] is the fp32 sum of that operand's
// row (bf16 pair dot products against ones on the VALU). A version whose
// waves ran apart through per-slot LDS counters instead of the barrier
// measured slower (waits for slot refills dominated).
//
// The ring and the staged weight rows are LDS written by the loads
// themselves, which the compiler cannot order against its own LDS reads: it
// would drain every load in flight before each read and each barrier. So
// the kernel reads them with explicit ds_read_b128 and orders them itself:
// a wave waits for its own loads of a fine (s_waitcnt vmcnt) before the
// barrier that publishes it, and for its reads (lgkmcnt) before using them.
constexpr int kRing = 4;
typedef __attribute__((address_space(3))) void lds_void_t;

template <int D>
struct StreamSmem {
  uint32_t bits[kBitWords];
  int pre[kBitWords];
  float wf[kRing][D];                // per slot: the fine's weights r(pw * sw), widened
  int ids[kGroupWaves][kMaxM];
  int uni[kMaxUnion];
  uint32_t mask[kMaxUnion / 4];
  int n_union;
  int erels[kGroupWaves];
};

// s_waitcnt with vmcnt <= N (expcnt and lgkmcnt not waited for).
template <int N>
TAO_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 16 bytes from LDS byte address `addr`, not waited for.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
TAO_DEV u32x4 lds_read16(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in
// order: a loop whose body needs its index as a constant.
template <typename F, int... I>
TAO_DEV void static_for_seq(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
TAO_DEV void static_for(F&& f) {
  static_for_seq(f, std::make_integer_sequence<int, N>{});
}
// The same at addr + OFF (the instruction's immediate offset, so one
// address register serves several reads).
template <int OFF>
TAO_DEV u32x4 lds_read16_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "16-bit LDS offset");
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
  return r;
}
// s_waitcnt lgkmcnt(0), tied to the values it makes ready (so nothing that
// reads them is scheduled above it).
TAO_DEV void wait_lds(u32x4& a) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a)::"memory"); }
TAO_DEV void wait_lds(u32x4& a, u32x4& b) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b)::"memory");
}
TAO_DEV void wait_lds(u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d)::"memory");
}
// s_waitcnt lgkmcnt(N): every LDS read but the newest N has landed, which
// covers the values tied to it when N reads were issued after them.
template <int N>
TAO_DEV void wait_lds_behind(u32x4& a, u32x4& b) {
  static_assert(N >= 0 && N < 16, "lgkmcnt is four bits");
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}
template <int N>
TAO_DEV void wait_lds_behind(u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
  static_assert(N >= 0 && N < 16, "lgkmcnt is four bits");
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N) : "memory");
}
TAO_DEV uint4 as_uint4(const u32x4& v) { return make_uint4(v.x, v.y, v.z, v.w); }
TAO_DEV void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
TAO_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

template <int D, bool COARSE, bool FEAT>
__global__ __launch_bounds__(kGroupThreads) void read_stream_kernel(ReadTilesParams p) {

  constexpr int KK = D / 16, ET = D / 32, CPR = D / 8;   // k-steps, e-tiles, chunks per row
  constexpr int CPT = D * CPR / (64 * kGroupWaves);      // 1 KB wave loads per fine and wave
  static_assert(CPT * 64 * kGroupWaves == D * CPR, "whole wave loads per fine");
  static_assert(kRing == 4, "two fines read while two load");
  __shared__ StreamSmem<D> sm;
  // The ring of staged C^T (swizzled rows); after the last pass, each wave's
  // fine and coarse tiles for the epilogue's transpose.
  constexpr int kRingElems = kRing * D * D, kEpiElems = kGroupWaves * 2 * 32 * D;
  __shared__ __attribute__((aligned(16))) bf16_t ring_mem[kRingElems > kEpiElems ? kRingElems
                                                                                 : kEpiElems];
  bf16_t (*ring)[D * D] = reinterpret_cast<bf16_t (*)[D * D]>(ring_mem);
  __shared__ __attribute__((aligned(16))) bf16_t pwsw[kRing][2][D];     // staged pw and sw rows
  // D = 128: the head's fusion parameters, widened, fpar[0][d][i] =
  // a[h][d][i] and fpar[1][d][i] = b[h][d][i], loaded at the start and read
  // by the epilogue (not for D = 64, whose LDS would then exceed half a CU's).
  constexpr bool kStageParams = D == 128;
  __shared__ __attribute__((aligned(16))) float fpar[2][kStageParams ? D * 3 : 4];
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  // Tiles in reverse plan order: the latest tiles read the most fines, so
  // they start first and the light early tiles fill the end of the launch.
  const int grp = (p.n_tiles + kGroupWaves - 1) / kGroupWaves - 1 - (int)blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const int t0 = grp * kGroupWaves;
  const int nt = min(kGroupWaves, p.n_tiles - t0);

  // This wave's tile.
  int q_first = 0, nq = 0, slot = 0, M = 0, erel = 0, fine_on = 0, cpages = 0;
  if (w < nt) {
    const int64_t* desc = p.tiles + 8 * (t0 + w);
    q_first = (int)desc[0]; nq = (int)desc[1]; slot = (int)desc[2]; M = (int)desc[3];
    erel = (int)desc[4]; fine_on = (int)desc[6];
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
  if (lane == 0) sm.erels[w] = reads ? erel : -1;
  for (int i = tid; kStageParams && i < 2 * D * 3; i += kGroupThreads) {
    const int which = i / (D * 3), d = (i % (D * 3)) / 3, j = i % 3;
    fpar[which][d * 3 + j] =
        which == 0 ? load_param(p.fa, p.f_dtype, h * p.fa_s[0] + d * p.fa_s[1] + j * p.fa_s[2])
                   : load_param(p.fb, p.f_dtype, h * p.fb_s[0] + d * p.fb_s[1] + j * p.fb_s[2]);
  }

  // ---- h of this wave's queries in fp32, in the MFMA A layout: lane (li, hl)
  // holds row q = li, channels d = 16 kk + 8 hl + j; rows past the tile are 0.
  float hf[KK][8];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
#pragma unroll
    for (int j = 0; j < 8; ++j) hf[kk][j] = 0.0f;
  if (reads) {
    const int q = li < nq ? li : nq - 1;
    const bf16_t* rq = p.rq.p + b * p.rq.sb + (int64_t)(q_first + q) * p.rq.st + h * p.rq.sh;
    float mx = -__builtin_inff();
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      unpack8f(*(const uint4*)(rq + 16 * kk + 8 * hl), hf[kk]);
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, hf[kk][j]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sum = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) { hf[kk][j] = __expf(hf[kk][j] - mx); sum += hf[kk][j]; }
    sum += __shfl_xor(sum, 32, 64);
    // h = r(softmax); it only shapes the read, never a route.
    const float inv = li < nq ? __builtin_amdgcn_rcpf(sum) : 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) hf[kk][j] = rbf(hf[kk][j] * inv);
  }
  // The same h as bf16 pairs (exact: h is rounded to bf16), channel 2 i of
  // the lane's eight in the low half of hp[kk][i]: the index-only read keeps
  // these instead of hf, which leaves registers for its operand pipeline.
  uint32_t hp[KK][4];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
#pragma unroll
    for (int i = 0; i < 4; ++i) hp[kk][i] = pack_bf16x2(hf[kk][2 * i], hf[kk][2 * i + 1]);

  // Feature writers: the mixture's normaliser for query li, the sum over the
  // wave's selected fines of mass = sum_d h[d] exp(z[d]) (fp32, the same
  // order as the per-fine mass of the read below).
  float tot = 0.0f;
  if constexpr (FEAT) {
    if (reads) {
      const int32_t* sel = p.sel_pool + ((size_t)slot * BH + bh) * p.sel_cap;
      const bf16_t* zb = p.fine_z + (size_t)bh * p.fine_cap * D;
      for (int m = 0; m < M; ++m) {
        const int fid = sel[m];
        float part = 0.0f;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          float zf[8];
          unpack8f(*(const uint4*)(zb + (size_t)fid * D + 16 * kk + 8 * hl), zf);
#pragma unroll
          for (int j = 0; j < 8; ++j) part += hf[kk][j] * expf(zf[j]);
        }
        part += __shfl_xor(part, 32, 64);
        tot += part;
      }
    }
  }

  floatx16 acc[ET];
#pragma unroll
  for (int t = 0; t < ET; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
  // den of query li, this lane's half of the channels: the fp32 sum of the
  // A operand's elements (bf16 pairs against ones on the VALU, which leaves
  // the matrix core to the numerator).
  float den_part = 0.0f;
  const bf16x2 ones2 = __builtin_bit_cast(bf16x2, 0x3F803F80u);

  const bf16_t* bank = p.bank + (size_t)bh * p.fine_cap * D * D;
  const bf16_t* sw_base = p.sw + (size_t)bh * p.fine_cap * D;
  __syncthreads();   // sm.erels

  // ---- one pass per distinct epoch of the group's reading tiles, ascending
  for (int pass_erel = -1;;) {
    int next = 0x7FFFFFFF;
#pragma unroll
    for (int v = 0; v < kGroupWaves; ++v) {
      const int e = sm.erels[v];
      if (e > pass_erel && e < next) next = e;
    }
    if (next == 0x7FFFFFFF) break;
    pass_erel = next;
    const bool in_pass = reads && erel == pass_erel;
    const int pass_epoch = p.first_epoch + pass_erel;
    const int sw_split = (pass_epoch / p.group) * p.group;
    const bf16_t* pw_base = p.pw_pool + ((size_t)pass_erel * BH + bh) * p.pool_pcap * D;
    const bf16_t* psw_base =
        p.psw_pool ? p.psw_pool + ((size_t)pass_erel * BH + bh) * 8 * D : nullptr;

    // ---- union of the pass's selected sets (ascending fine id), per-wave masks
    for (int i = tid; i < kBitWords; i += kGroupThreads) sm.bits[i] = 0;
    for (int i = tid; i < kMaxUnion / 4; i += kGroupThreads) sm.mask[i] = 0;
    if (in_pass) {
      const int32_t* sel = p.sel_pool + ((size_t)slot * BH + bh) * p.sel_cap;
      for (int m = lane; m < M; m += 64) sm.ids[w][m] = sel[m];
    }
    __syncthreads();
    if (in_pass)
      for (int m = lane; m < M; m += 64) {
        const int id = sm.ids[w][m];
        atomicOr(&sm.bits[id >> 5], 1u << (id & 31));
      }
    __syncthreads();
    if (w == 0) {
      constexpr int WPL = kBitWords / 64;
      int cnt[WPL], total = 0;
#pragma unroll
      for (int i = 0; i < WPL; ++i) {
        cnt[i] = __popc(sm.bits[lane * WPL + i]);
        total += cnt[i];
      }
      int incl = total;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off, 64);
        if (lane >= off) incl += v;
      }
      int run = incl - total;
#pragma unroll
      for (int i = 0; i < WPL; ++i) { sm.pre[lane * WPL + i] = run; run += cnt[i]; }
      if (lane == 63) sm.n_union = incl;
    }
    __syncthreads();
    for (int i = tid; i < kBitWords; i += kGroupThreads) {
      uint32_t bits = sm.bits[i];
      int r = sm.pre[i];
      while (bits) {
        sm.uni[r++] = i * 32 + __ffs(bits) - 1;
        bits &= bits - 1;
      }
    }
    if (in_pass)
      for (int m = lane; m < M; m += 64) {
        const int id = sm.ids[w][m];
        const uint32_t word = sm.bits[id >> 5];
        const int rank = sm.pre[id >> 5] + __popc(word & ((1u << (id & 31)) - 1u));
        atomicOr(&sm.mask[rank >> 2], 1u << ((rank & 3) * 8 + w));
      }
    __syncthreads();
    const int U = sm.n_union;

    // ---- stream the union through the ring
    auto issue = [&](int f) __attribute__((always_inline)) {
      const int s = f % kRing;
      const int fid = sm.uni[f];
      const bf16_t* base = bank + (size_t)fid * D * D;
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int J = w * CPT + i;            // this wave's 1 KB block of the slot
        const int L = J * 64 + lane;          // 16-byte chunk index in the slot
        const int row = L / CPR, pos = L % CPR;
        __builtin_amdgcn_global_load_lds(base + (size_t)row * D + (pos ^ (row % CPR)) * 8,
                                         (lds_void_t*)(&ring[s][0] + J * 64 * 8), 16, 0, 0);
      }
      if (FEAT && w == 0 && lane < CPR) {
        const bf16_t* src = p.fine_z + ((size_t)bh * p.fine_cap + fid) * D + lane * 8;
        __builtin_amdgcn_global_load_lds(src, (lds_void_t*)&pwsw[s][0][0], 16, 0, 0);
      } else if (!FEAT && w == 0 && lane < 2 * CPR) {
        const bf16_t* src =
            lane < CPR ? pw_base + (size_t)(fid / p.group) * D + lane * 8
                       : (fid < sw_split ? sw_base + (size_t)fid * D
                                         : psw_base + (size_t)(fid - sw_split) * D) +
                             (lane - CPR) * 8;
        __builtin_amdgcn_global_load_lds(src, (lds_void_t*)&pwsw[s][0][0], 16, 0, 0);
      }
    };
    // Wave 0 turns the fine's pw and sw rows into its weights.
    auto make_wr = [&](int f) __attribute__((always_inline)) {
      const int s = f % kRing;
      if (FEAT && w == 0 && lane < CPR) {
        // Feature writers: exp(z) of the fine's descriptor.
        u32x4 zv = lds_read16(lds_addr(&pwsw[s][0][lane * 8]));
        wait_lds(zv);
        float wv[8];
        unpack8f(as_uint4(zv), wv);
#pragma unroll
        for (int j = 0; j < 8; ++j) wv[j] = expf(wv[j]);
        *(float4*)&sm.wf[s][lane * 8] = make_float4(wv[0], wv[1], wv[2], wv[3]);
        *(float4*)&sm.wf[s][lane * 8 + 4] = make_float4(wv[4], wv[5], wv[6], wv[7]);
      } else if (!FEAT && w == 0 && lane < CPR) {
        u32x4 pwv = lds_read16(lds_addr(&pwsw[s][0][lane * 8]));
        u32x4 swv = lds_read16(lds_addr(&pwsw[s][1][lane * 8]));
        wait_lds(pwv, swv);
        float wv[8];
        unpack8f(slice_weights(as_uint4(pwv), as_uint4(swv)), wv);
        *(float4*)&sm.wf[s][lane * 8] = make_float4(wv[0], wv[1], wv[2], wv[3]);
        *(float4*)&sm.wf[s][lane * 8 + 4] = make_float4(wv[4], wv[5], wv[6], wv[7]);
      }
    };
    // Feature writers: coef = r(mix * h) with mix = mass / tot of this fine
    // (feature_read_coefficients), read against C^T with no denominator.
    auto consume_feat = [&](int u) __attribute__((always_inline)) {
      if (!(in_pass && ((sm.mask[u >> 2] >> ((u & 3) * 8 + w)) & 1u))) return;
      const int s = u % kRing;
      const uint32_t cs = lds_addr(&ring[s][0]);
      float part = 0.0f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const float4 e0 = *(const float4*)&sm.wf[s][16 * kk + 8 * hl];
        const float4 e1 = *(const float4*)&sm.wf[s][16 * kk + 8 * hl + 4];
        const float ev[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) part += hf[kk][j] * ev[j];
      }
      part += __shfl_xor(part, 32, 64);
      const float mix = part / tot;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int c = 2 * kk + hl;
        u32x4 bq[ET];
#pragma unroll
        for (int t = 0; t < ET; ++t) {
          const int row = 32 * t + li;
          bq[t] = lds_read16(cs + (uint32_t)(row * D + 8 * (c ^ (row % CPR))) * 2);
        }
        const bf16x8 a = as_bf16x8(make_uint4(
            pack_bf16x2(mix * hf[kk][0], mix * hf[kk][1]), pack_bf16x2(mix * hf[kk][2], mix * hf[kk][3]),
            pack_bf16x2(mix * hf[kk][4], mix * hf[kk][5]), pack_bf16x2(mix * hf[kk][6], mix * hf[kk][7])));
        if constexpr (ET == 4) wait_lds(bq[0], bq[1], bq[2], bq[3]);
        else wait_lds(bq[0], bq[1]);
#pragma unroll
        for (int t = 0; t < ET; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(as_uint4(bq[t])), a, acc[t],
                                                           0, 0, 0);
      }
    };
    auto consume = [&](int u) __attribute__((always_inline)) {
      if (!(in_pass && ((sm.mask[u >> 2] >> ((u & 3) * 8 + w)) & 1u))) return;
      const int s = u % kRing;
      const uint32_t cs = lds_addr(&ring[s][0]);
      const uint32_t ws = lds_addr(&sm.wf[s][8 * hl]);
      // Step kk runs the ET MFMAs of k-step kk and, between them, builds the
      // A operand of step kk + 1 (r(h * w), two channels per MFMA gap) and
      // adds step kk's operand into den, so the VALU work issues while the
      // matrix core is busy. Operands are read two steps ahead: stage kk is
      // step kk's C^T rows and step kk + 1's weights.
      //
      // Row e = 32 t + li keeps logical chunk c at c ^ (e % CPR) = c ^ (li % CPR)
      // (32 t is a multiple of CPR), so one address per step serves every t
      // through the read's immediate offset.
      static_assert(32 % CPR == 0, "row swizzle independent of the e-tile");
      const uint32_t rowb = cs + (uint32_t)(li * D) * 2;
      auto read_c = [&](auto kkc, u32x4(&bq)[ET]) __attribute__((always_inline)) {
        constexpr int kk = decltype(kkc)::value;
        const uint32_t at = rowb + (uint32_t)((2 * kk + hl) ^ (li % CPR)) * 16;
        bq[0] = lds_read16_at<0>(at);
        bq[1] = lds_read16_at<32 * D * 2>(at);
        if constexpr (ET == 4) {
          bq[2] = lds_read16_at<64 * D * 2>(at);
          bq[3] = lds_read16_at<96 * D * 2>(at);
        }
      };
      auto read_w = [&](auto kkc, u32x4& w0, u32x4& w1) __attribute__((always_inline)) {
        constexpr int kk = decltype(kkc)::value;
        w0 = lds_read16_at<64 * kk>(ws);
        w1 = lds_read16_at<64 * kk + 16>(ws);
      };
      // Stage kk's reads: the rows, then the next step's weights if any.
      auto stage = [&](auto kkc, u32x4(&bq)[ET], u32x4& w0, u32x4& w1) __attribute__((always_inline)) {
        constexpr int kk = decltype(kkc)::value;
        read_c(kkc, bq);
        if constexpr (kk + 1 < KK) read_w(std::integral_constant<int, kk + 1>{}, w0, w1);
      };
      auto stage_reads = [](int kk) constexpr { return ET + (kk + 1 < KK ? 2 : 0); };
      // Channel pair i of step kk's A operand.
      auto a_pair = [&](int kk, int i, const u32x4& w0, const u32x4& w1) __attribute__((always_inline)) {
        const u32x4& wv = i < 2 ? w0 : w1;
        const uint32_t x = (i & 1) ? wv.z : wv.x, y = (i & 1) ? wv.w : wv.y;
        const uint32_t hv = hp[kk][i];
        return pack_bf16x2(__uint_as_float(hv << 16) * __uint_as_float(x),
                           __uint_as_float(hv & 0xFFFF0000u) * __uint_as_float(y));
      };

      // hp is loop-invariant: left visible, the compiler hoists its
      // unpacking out of the fine loop and holds all of hf again.
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        asm volatile("" : "+v"(hp[kk][0]), "+v"(hp[kk][1]), "+v"(hp[kk][2]), "+v"(hp[kk][3]));
      uint32_t a_cur[4];
      {
        u32x4 w0, w1;
        read_w(std::integral_constant<int, 0>{}, w0, w1);
        wait_lds(w0, w1);
#pragma unroll
        for (int i = 0; i < 4; ++i) a_cur[i] = a_pair(0, i, w0, w1);
      }
      u32x4 c0[ET], v0a, v0b, c1[ET], v1a, v1b;
      stage(std::integral_constant<int, 0>{}, c0, v0a, v0b);
      if constexpr (KK > 1) stage(std::integral_constant<int, 1>{}, c1, v1a, v1b);
      static_for<KK>([&](auto kkc) __attribute__((always_inline)) {
        constexpr int kk = decltype(kkc)::value;
        // Stage kk has landed when only stage kk + 1's reads are in flight.
        constexpr int behind = kk + 1 < KK ? stage_reads(kk + 1) : 0;
        if constexpr (ET == 4) wait_lds_behind<behind>(c0[0], c0[1], c0[2], c0[3]);
        else wait_lds_behind<behind>(c0[0], c0[1]);
        wait_lds_behind<behind>(v0a, v0b);
        u32x4 c2[ET], v2a, v2b;
        if constexpr (kk + 2 < KK) stage(std::integral_constant<int, kk + 2>{}, c2, v2a, v2b);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t a_next[4];
        const bf16x8 a = as_bf16x8(make_uint4(a_cur[0], a_cur[1], a_cur[2], a_cur[3]));
#pragma unroll
        for (int t = 0; t < ET; ++t) {
          // num^T[e][q]: the C^T rows are the A operand, so lane li ends up
          // holding query li.
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(as_uint4(c0[t])), a, acc[t],
                                                           0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = t * 4 / ET; i < (t + 1) * 4 / ET; ++i)
            if constexpr (kk + 1 < KK) a_next[i] = a_pair(kk + 1, i, v0a, v0b);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
          den_part = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a_cur[i]), ones2,
                                                     den_part, false);
        if constexpr (kk + 1 < KK) {
#pragma unroll
          for (int i = 0; i < 4; ++i) a_cur[i] = a_next[i];
#pragma unroll
          for (int t = 0; t < ET; ++t) c0[t] = c1[t];
          v0a = v1a;
          v0b = v1b;
        }
        if constexpr (kk + 2 < KK) {
#pragma unroll
          for (int t = 0; t < ET; ++t) c1[t] = c2[t];
          v1a = v2a;
          v1b = v2b;
        }
      });
    };
    // Barrier that publishes the ring: the caller has waited for its own
    // loads; the weights written by wave 0 are ordinary LDS stores.
    auto ring_barrier = [&]() __attribute__((always_inline)) {
      wait_lds();
      __builtin_amdgcn_s_barrier();
    };
    // Fines go in pairs, one barrier per pair: pair (u, u + 1) is read from
    // ring slots u % 4 and (u + 1) % 4 while fines u + 2 and u + 3 load into
    // the two slots the previous pair freed. A wave's time per barrier is
    // then its consume of two fines, and the two fines' slowest waves are
    // often different ones.
    for (int f = 0; f < min(U, 2); ++f) issue(f);
    wait_vmcnt<0>();
    for (int f = 0; f < min(U, 2); ++f) make_wr(f);
    ring_barrier();
    for (int u = 0; u < U; u += 2) {
      // A wave that reads fine u issues after it: the other waves' issues
      // have just filled the memory pipeline.
      if constexpr (FEAT) consume_feat(u);
      else consume(u);
      for (int f = u + 2; f < min(U, u + 4); ++f) issue(f);
      if (u + 1 < U) {
        if constexpr (FEAT) consume_feat(u + 1);
        else consume(u + 1);
      }
      wait_vmcnt<0>();        // this wave's loads of fines u + 2 and u + 3
      for (int f = u + 2; f < min(U, u + 4); ++f) make_wr(f);
      ring_barrier();
    }
    wait_vmcnt<0>();
    __syncthreads();   // the next pass's setup
  }

  // ---- epilogue: fine = r(r(num) / r(den)), the coarse read, the fusion.
  // Lane li holds query li's values for e = 32 t + 8 g + 4 hl + (0..3). They
  // go through this wave's part of the (now idle) ring as [q][e] tiles whose
  // 16-byte units are XOR-swizzled by the row, so the fusion reads whole
  // 8-channel units and loads and stores 16 bytes per lane.
  if (!reads) return;
  const bool coarse_on = COARSE && cpages >= 1;
  const bf16_t* gc = coarse_on && !FEAT
                         ? p.coarse_pool + ((size_t)(cpages - p.coarse_first) * BH + bh) * D * D
                         : nullptr;
  bf16_t* tile_f = ring_mem + (size_t)w * 2 * 32 * D;
  bf16_t* tile_c = tile_f + 32 * D;
  const float den = den_part + __shfl_xor(den_part, 32, 64);
  const float rden = __builtin_amdgcn_rcpf(rbf(den));
  if (p.save_fine && hl == 0 && li < nq) p.save_den[((size_t)b * p.T + q_first + li) * p.H + h] = rbf(den);
  auto unit_at = [&](int row, int unit) __attribute__((always_inline)) {
    return row * D + 8 * (unit ^ (row % CPR));
  };
#pragma unroll
  for (int t = 0; t < ET; ++t) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int at = unit_at(li, 4 * t + g) + 4 * hl;
      float f[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        f[k] = FEAT ? rbf(acc[t][4 * g + k]) : rbf(rbf(acc[t][4 * g + k]) * rden);
      *(uint2*)&tile_f[at] = make_uint2(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]));
    }
    if constexpr (COARSE && !FEAT) {
      if (coarse_on) {
        floatx16 cacc;
#pragma unroll
        for (int i = 0; i < 16; ++i) cacc[i] = 0.0f;
        uint4 gb[KK];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          gb[kk] = *(const uint4*)(gc + (size_t)(32 * t + li) * D + 16 * kk + 8 * hl);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          const bf16x8 a = as_bf16x8(make_uint4(hp[kk][0], hp[kk][1], hp[kk][2], hp[kk][3]));
          cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(gb[kk]), a, cacc, 0, 0, 0);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *(uint2*)&tile_c[unit_at(li, 4 * t + g) + 4 * hl] =
              make_uint2(pack_bf16x2(cacc[4 * g], cacc[4 * g + 1]),
                         pack_bf16x2(cacc[4 * g + 2], cacc[4 * g + 3]));
      }
    }
  }
  if constexpr (COARSE && FEAT) {
    // Feature writers' coarse read (tao_stream.py:301-305): the mixture of
    // the chunk's completed pages, coef = r(mass_p / sum_p mass_p * h) with
    // mass_p = sum_d h[d] exp(page_z[p][d]) in fp32, against each page's C^T.
    if (coarse_on) {
      const bf16_t* pzb = p.page_z + (size_t)bh * p.page_cap * D;
      const bf16_t* pcb = p.page_c + (size_t)bh * p.page_cap * D * D;
      auto page_mass = [&](int pg) __attribute__((always_inline)) {
        float part = 0.0f;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          float zf[8];
          unpack8f(*(const uint4*)(pzb + (size_t)pg * D + 16 * kk + 8 * hl), zf);
#pragma unroll
          for (int j = 0; j < 8; ++j) part += hf[kk][j] * expf(zf[j]);
        }
        return part + __shfl_xor(part, 32, 64);
      };
      float totc = 0.0f;
      for (int pg = 0; pg < cpages; ++pg) totc += page_mass(pg);
      floatx16 cacc[ET];
#pragma unroll
      for (int t = 0; t < ET; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) cacc[t][i] = 0.0f;
      for (int pg = 0; pg < cpages; ++pg) {
        const float mix = page_mass(pg) / totc;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          const bf16x8 a = as_bf16x8(make_uint4(
              pack_bf16x2(mix * hf[kk][0], mix * hf[kk][1]), pack_bf16x2(mix * hf[kk][2], mix * hf[kk][3]),
              pack_bf16x2(mix * hf[kk][4], mix * hf[kk][5]), pack_bf16x2(mix * hf[kk][6], mix * hf[kk][7])));
#pragma unroll
          for (int t = 0; t < ET; ++t) {
            const uint4 gb =
                *(const uint4*)(pcb + ((size_t)pg * D + 32 * t + li) * D + 16 * kk + 8 * hl);
            cacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(gb), a, cacc[t], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int t = 0; t < ET; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *(uint2*)&tile_c[unit_at(li, 4 * t + g) + 4 * hl] =
              make_uint2(pack_bf16x2(cacc[t][4 * g], cacc[t][4 * g + 1]),
                         pack_bf16x2(cacc[t][4 * g + 2], cacc[t][4 * g + 3]));
    }
  }
  if constexpr (kStageParams)
    fuse_rows<D, COARSE, true>(p, fpar, tile_f, tile_c, lane, b, h, q_first, nq, coarse_on);
  else
    fuse_rows<D, COARSE, false>(p, nullptr, tile_f, tile_c, lane, b, h, q_first, nq, coarse_on);
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
  hipLaunchKernelGGL((read_groups_kernel<D_, C_, Q_, false>), grid, dim3(kGroupThreads), 0, s, p)
#define TAO_MIXTURE_LAUNCH(D_, C_)                                                            \
  hipLaunchKernelGGL((read_groups_kernel<D_, C_, true, true>), grid, dim3(kGroupThreads), 0, s, p)
#define TAO_STREAM_LAUNCH(D_, C_)                                                             \
  hipLaunchKernelGGL((read_stream_kernel<D_, C_, false>), grid, dim3(kGroupThreads), 0, s, p)
#define TAO_FEATURE_LAUNCH(D_, C_)                                                            \
  hipLaunchKernelGGL((read_stream_kernel<D_, C_, true>), grid, dim3(kGroupThreads), 0, s, p)
  if (head_dim != 128 && head_dim != 64) return hipErrorInvalidValue;
  if (p.fine_z) {
    // Feature writers, no saves: per-query routes index-only; turn routes
    // with or without the page mixture (page_c). Saves (the backward's
    // pre-fusion heads) only with per-query routes.
    if (p.save_fine && !perq) return hipErrorInvalidValue;
    const bool pages = p.page_c != nullptr;
    if (perq) {
      if (coarse || (pages && !p.page_z)) return hipErrorInvalidValue;
      if (pages) {
        if (head_dim == 128) TAO_MIXTURE_LAUNCH(128, true); else TAO_MIXTURE_LAUNCH(64, true);
      } else {
        if (head_dim == 128) TAO_MIXTURE_LAUNCH(128, false); else TAO_MIXTURE_LAUNCH(64, false);
      }
    } else if (pages) {
      if (!p.page_z) return hipErrorInvalidValue;
      if (head_dim == 128) TAO_FEATURE_LAUNCH(128, true); else TAO_FEATURE_LAUNCH(64, true);
    } else {
      if (coarse) return hipErrorInvalidValue;
      if (head_dim == 128) TAO_FEATURE_LAUNCH(128, false); else TAO_FEATURE_LAUNCH(64, false);
    }
    return hipGetLastError();
  }
  if (head_dim == 128) {
    if (perq) {
      if (coarse) TAO_READ_LAUNCH(128, true, true); else TAO_READ_LAUNCH(128, false, true);
    } else {
      if (coarse) TAO_STREAM_LAUNCH(128, true); else TAO_STREAM_LAUNCH(128, false);
    }
  } else {
    if (perq) {
      if (coarse) TAO_READ_LAUNCH(64, true, true); else TAO_READ_LAUNCH(64, false, true);
    } else {
      if (coarse) TAO_STREAM_LAUNCH(64, true); else TAO_STREAM_LAUNCH(64, false);
    }
  }
#undef TAO_READ_LAUNCH
#undef TAO_STREAM_LAUNCH
  return hipGetLastError();
}

}  // namespace tao
