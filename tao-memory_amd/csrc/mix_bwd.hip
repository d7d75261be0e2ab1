// Backward of the feature writers' full-sequence read for gfx950: the
// adjoints the reference takes by autograd through feature_read_coefficients
// and selected_fine_numerator (association_writer.py:46-53,
// indirect_fine.py:65-120, tao_stream.py:600-662), the descriptors
// z = r(log mass) (tao_stream.py:80-97, 543-549) and the structured-Gram
// matrix (structured_writer.py:16-34). Gradients are those of the forward's
// function at the forward's values and selections; accumulation is fp32,
// MFMA operands are bf16.
#include <algorithm>

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

// Items (fines or pages) of the query block starting at q0: fines visible to
// its tile, or the tile's completed pages once the block reads the coarse
// branch.
TAO_DEV int block_items(const MixBwdParams& p, int q0) {
  const int lag = p.keep / p.ft;
  const int tile = q0 / p.ft;
  const int V = tile > lag ? tile - lag : 0;
  if (q0 < p.first_query) return 0;
  return p.qsel ? V : V / p.group;
}

// ---------------------------------------------------------------------------
// Query-major pass. One workgroup per (32 queries, batch, head), D / 32 waves;
// wave w owns channels 32 w .. 32 w + 31. Over the union of the block's items
// (ascending), the masses give w_m; then per item its C (staged as [d][e]) and
// dch = dout C^T by v_mfma_f32_32x32x16_bf16 (A = the block's dout rows, lane
// = channel d, rows = queries), accumulating dh and dw_m; finally dmass_m and
// its exp(z_m) term of dh. w_m and dmass_m go to wv / dmv for the item pass.
template <int D>
struct MixQSmem {
  bf16_t c[D][D + 8];                 // C of the current item: [d][e]
  float hq[32][D + 1];                // the block's h (fp32)
  float ez[D];                        // exp(z) of the current item
  uint32_t qw[32][16];                // per query selection words (fine items)
  float wl[32][kMixMaxRank];          // mass, then w, per query and rank
  float dwl[32][kMixMaxRank];         // dw, then dmass
  float tot[32], S[32], dwtmp[32];
  int run[32], cnt[32];
  int uni[kMixMaxItems];
  int n_union;
};

template <int D>
__global__ __launch_bounds__(2 * D) void mix_query_bwd_kernel(MixBwdParams p) {
  constexpr int NT = 2 * D, KK = D / 16, TPQ = NT / 32;   // TPQ threads per query (16 channels)
  __shared__ MixQSmem<D> sm;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int b = bh / p.H, h = bh % p.H;
  const int q0 = (blockIdx.x / BH) * 32;
  if (q0 >= p.T) return;
  const int V = block_items(p, q0);
  if (V <= 0) return;
  const bool fine = p.qsel != nullptr;
  const int nq = min(32, p.T - q0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const int words = (V + 31) >> 5;
  auto row_of = [&](int q) { return (((size_t)b * p.T + q0 + q) * p.H + h); };
  for (int i = tid; i < 32 * D; i += NT) {
    const int q = i / D, d = i % D;
    sm.hq[q][d] = q < nq ? bf2f(p.h[row_of(q) * D + d]) : 0.0f;
  }
  if (fine) {
    for (int i = tid; i < 32 * 16; i += NT) {
      const int q = i / 16, wd = i % 16;
      uint32_t bits = 0;
      if (q < nq && wd < words) {
        bits = p.qsel[row_of(q) * p.qsel_words + wd];
        const int lo = wd * 32;
        if (V - lo < 32) bits &= (1u << (V - lo)) - 1u;
      }
      sm.qw[q][wd] = bits;
    }
  }
  if (tid < 32) {
    sm.tot[tid] = 0.0f;
    sm.S[tid] = 0.0f;
    sm.dwtmp[tid] = 0.0f;
    sm.run[tid] = 0;
  }
  __syncthreads();
  if (tid == 0) {
    int n = 0;
    if (fine) {
      for (int wd = 0; wd < words; ++wd) {
        uint32_t u = 0;
        for (int q = 0; q < 32; ++q) u |= sm.qw[q][wd];
        while (u) {
          sm.uni[n++] = wd * 32 + __ffs(u) - 1;
          u &= u - 1;
        }
      }
    } else {
      for (int m = 0; m < V; ++m) sm.uni[n++] = m;
    }
    sm.n_union = n;
  }
  if (tid < 32) {
    int c = 0;
    if (fine) {
      for (int wd = 0; wd < words; ++wd) c += __popc(sm.qw[tid][wd]);
    } else {
      c = tid < nq ? V : 0;
    }
    sm.cnt[tid] = c;
  }
  __syncthreads();
  const int U = sm.n_union;
  auto selects = [&](int q, int id) __attribute__((always_inline)) {
    return fine ? ((sm.qw[q][id >> 5] >> (id & 31)) & 1u) != 0 : q < nq;
  };
  const bf16_t* zb = p.z + (size_t)bh * p.cap * D;
  const bf16_t* mb = p.mats + (size_t)bh * p.cap * D * D;

  // ---- masses: thread (q = tid / TPQ, part) sums 16 channels
  {
    const int q = tid / TPQ, part = tid % TPQ;
    int rank = 0;
    for (int u = 0; u < U; ++u) {
      const int id = sm.uni[u];
      for (int d = tid; d < D; d += NT) sm.ez[d] = __expf(bf2f(zb[(size_t)id * D + d]));
      __syncthreads();
      float m = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) m += sm.hq[q][16 * part + j] * sm.ez[16 * part + j];
#pragma unroll
      for (int off = 1; off < TPQ; off <<= 1) m += __shfl_xor(m, off, 64);
      if (part == 0 && selects(q, id)) {
        if (rank < kMixMaxRank) sm.wl[q][rank] = m;
        sm.tot[q] += m;
        ++rank;
      }
      __syncthreads();
    }
  }
  for (int i = tid; i < 32 * kMixMaxRank; i += NT) {
    const int q = i / kMixMaxRank, r = i % kMixMaxRank;
    if (r < min(sm.cnt[q], p.R)) sm.wl[q][r] = sm.wl[q][r] / sm.tot[q];
  }
  // ---- dout rows of the block as the bf16 A operand (row li, k = e)
  uint4 ad[KK];
  {
    const int q = li < nq ? li : nq - 1;
    const float* dr = p.dout + row_of(q) * D;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const float4 x0 = *(const float4*)(dr + 16 * kk + 8 * hl);
      const float4 x1 = *(const float4*)(dr + 16 * kk + 8 * hl + 4);
      const float s = li < nq ? 1.0f : 0.0f;
      ad[kk] = make_uint4(pack_bf16x2(s * x0.x, s * x0.y), pack_bf16x2(s * x0.z, s * x0.w),
                          pack_bf16x2(s * x1.x, s * x1.y), pack_bf16x2(s * x1.z, s * x1.w));
    }
  }
  const int d = 32 * w + li;
  float hv[16], dh_acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int q = 8 * (i / 4) + 4 * hl + (i % 4);
    hv[i] = sm.hq[q][d];
    dh_acc[i] = 0.0f;
  }
  __syncthreads();
  // ---- per item: dch = dout C^T, then dh and dw
  for (int u = 0; u < U; ++u) {
    const int id = sm.uni[u];
    const bf16_t* ct = mb + (size_t)id * D * D;
    // stage C[d][e] = C^T[e][d]: thread pairs of rows e, e + 1 and 8 channels
    for (int job = tid; job < (D / 2) * (D / 8); job += NT) {
      const int e0 = 2 * (job % (D / 2)), ch = job / (D / 2);
      const uint4 ua = *(const uint4*)(ct + (size_t)e0 * D + ch * 8);
      const uint4 ub = *(const uint4*)(ct + (size_t)(e0 + 1) * D + ch * 8);
      const uint32_t wa[4] = {ua.x, ua.y, ua.z, ua.w}, wb[4] = {ub.x, ub.y, ub.z, ub.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *(uint32_t*)&sm.c[ch * 8 + 2 * i][e0] = (wa[i] & 0xFFFFu) | (wb[i] << 16);
        *(uint32_t*)&sm.c[ch * 8 + 2 * i + 1][e0] = (wa[i] >> 16) | (wb[i] & 0xFFFF0000u);
      }
    }
    __syncthreads();
    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          as_bf16x8(ad[kk]), as_bf16x8(*(const uint4*)&sm.c[d][16 * kk + 8 * hl]), acc, 0, 0, 0);
    float part[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int q = 8 * (i / 4) + 4 * hl + (i % 4);
      const bool s = selects(q, id);
      const float wq = s ? sm.wl[q][min(sm.run[q], kMixMaxRank - 1)] : 0.0f;
      dh_acc[i] += acc[i] * wq;
      part[i] = s ? acc[i] * hv[i] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) part[i] += __shfl_xor(part[i], off, 64);
    if (li == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) atomicAdd(&sm.dwtmp[8 * (i / 4) + 4 * hl + (i % 4)], part[i]);
    }
    __syncthreads();
    if (tid < 32 && selects(tid, id)) {
      const int r = min(sm.run[tid], kMixMaxRank - 1);
      const float dw = sm.dwtmp[tid];
      sm.dwl[tid][r] = dw;
      sm.S[tid] += dw * sm.wl[tid][r];
      sm.run[tid] = r + 1;
    }
    if (tid < 32) sm.dwtmp[tid] = 0.0f;
    __syncthreads();
  }
  // ---- dmass, and the saves for the item pass
  for (int i = tid; i < 32 * kMixMaxRank; i += NT) {
    const int q = i / kMixMaxRank, r = i % kMixMaxRank;
    if (q < nq && r < min(sm.cnt[q], p.R)) {
      const float dm = (sm.dwl[q][r] - sm.S[q]) / sm.tot[q];
      sm.dwl[q][r] = dm;
      p.wv[row_of(q) * p.R + r] = sm.wl[q][r];
      p.dmv[row_of(q) * p.R + r] = dm;
    }
  }
  __syncthreads();
  // ---- dh += sum_m dmass_m exp(z_m)
  int rk[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) rk[i] = 0;
  for (int u = 0; u < U; ++u) {
    const int id = sm.uni[u];
    const float ez = __expf(bf2f(zb[(size_t)id * D + d]));
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int q = 8 * (i / 4) + 4 * hl + (i % 4);
      if (selects(q, id)) {
        dh_acc[i] += sm.dwl[q][min(rk[i], kMixMaxRank - 1)] * ez;
        ++rk[i];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int q = 8 * (i / 4) + 4 * hl + (i % 4);
    if (q < nq) p.dh[row_of(q) * D + d] += dh_acc[i];
  }
}

// ---------------------------------------------------------------------------
// Item-major pass. One 256-thread workgroup per (item, batch, head): over the
// queries that can read the item, in chunks of 32, dC^T[e][d] = sum_q
// dout[q][e] r(w_q h[q][d]) (A = dout^T chunk [e][q], B = channel^T chunk
// [d][q], both staged in LDS; only queries that read the item contribute)
// and dz[d] = exp(z[d]) sum_q dmass_q h[q][d].
template <int D>
struct MixISmem {
  bf16_t xt[D][40];                   // dout^T [e][q]
  bf16_t yt[D][40];                   // channel^T [d][q]
  float wq[32], dmq[32];
};

template <int D>
__global__ __launch_bounds__(256) void mix_item_bwd_kernel(MixBwdParams p) {
  constexpr int NTI = D / 32, TILES = NTI * NTI, TPW = (TILES + 3) / 4;
  __shared__ MixISmem<D> sm;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int item = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const bool fine = p.qsel != nullptr;
  const int lag = p.keep / p.ft;
  // First tile that reads the item: V > item (fines) or V / group > item.
  const int t_first = fine ? item + lag + 1 : (item + 1) * p.group + lag;
  const int q_begin = max(p.first_query, t_first * p.ft);
  floatx16 acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
  float dzacc = 0.0f;
  auto row_of = [&](int q) { return (((size_t)b * p.T + q) * p.H + h); };
  for (int c0 = q_begin; c0 < p.T; c0 += 32) {
    int reads = 0;
    if (tid < 32) {
      const int q = c0 + tid;
      float wv = 0.0f, dm = 0.0f;
      if (q < p.T && block_items(p, q - q % 32) > item) {
        int rank = item;
        bool s = true;
        if (fine) {
          const uint32_t* qw = p.qsel + row_of(q) * p.qsel_words;
          s = ((qw[item >> 5] >> (item & 31)) & 1u) != 0;
          rank = 0;
          for (int wd = 0; wd < (item >> 5); ++wd) rank += __popc(qw[wd]);
          rank += __popc(qw[item >> 5] & ((1u << (item & 31)) - 1u));
        }
        if (s && rank < p.R) {
          wv = p.wv[row_of(q) * p.R + rank];
          dm = p.dmv[row_of(q) * p.R + rank];
        } else {
          s = false;
        }
        reads = s ? 1 : 0;
      }
      sm.wq[tid] = wv;
      sm.dmq[tid] = dm;
    }
    // publishes wq / dmq; chunks no query of which reads the item are skipped
    if (!__syncthreads_or(reads)) continue;
    for (int i = tid; i < 32 * D; i += 256) {
      const int q = i / D, e = i % D;
      const int tq = c0 + q;
      const bool live = tq < p.T && sm.wq[q] != 0.0f;
      const size_t row = row_of(live ? tq : c0);
      sm.xt[e][q] = f2bf(live ? p.dout[row * D + e] : 0.0f);
      sm.yt[e][q] = f2bf(live ? sm.wq[q] * bf2f(p.h[row * D + e]) : 0.0f);
    }
    if (tid < D) {
      float s = 0.0f;
      for (int q = 0; q < 32; ++q) {
        const int tq = c0 + q;
        if (tq < p.T && sm.dmq[q] != 0.0f) s += sm.dmq[q] * bf2f(p.h[row_of(tq) * D + tid]);
      }
      dzacc += s;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int tile = w * TPW + t;
      if (tile < TILES) {
        const int te = tile / NTI, td = tile % NTI;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              as_bf16x8(*(const uint4*)&sm.xt[32 * te + li][16 * kk + 8 * hl]),
              as_bf16x8(*(const uint4*)&sm.yt[32 * td + li][16 * kk + 8 * hl]), acc[t], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  float* out = p.dmat + ((size_t)bh * p.n_items + item) * D * D;
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int tile = w * TPW + t;
    if (tile < TILES) {
      const int te = tile / NTI, td = tile % NTI;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int e = 32 * te + 8 * (i / 4) + 4 * hl + (i % 4);
        out[(size_t)e * D + 32 * td + li] = acc[t][i];
      }
    }
  }
  if (tid < D) {
    const float ez = __expf(bf2f(p.z[((size_t)bh * p.cap + item) * D + tid]));
    p.dz[((size_t)bh * p.n_items + item) * D + tid] = dzacc * ez;
  }
}

// ---------------------------------------------------------------------------
// d mass per fine (see launch_mass_grad). Thread per (mat, d).
__global__ __launch_bounds__(256) void mass_grad_kernel(const float* dz, const float* dpz,
                                                        const float* mass, const float* extra,
                                                        float* dmass, int fines, int pages,
                                                        int group, int B, int H, int D) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)fines * B * H * D;
  if (i >= total) return;
  const int d = (int)(i % D);
  const size_t mat = i / D;                      // (f, b, h)
  const int f = (int)(mat / ((size_t)B * H));
  const int bh = (int)(mat % ((size_t)B * H));
  const int b = bh / H, h = bh % H;
  float g = dz[((size_t)bh * fines + f) * D + d] / mass[i];
  const int pg = f / group;
  if (pg < pages) {
    float pm = 0.0f;
    for (int j = 0; j < group; ++j)
      pm += mass[(((size_t)(pg * group + j) * B + b) * H + h) * D + d];
    g += dpz[((size_t)bh * pages + pg) * D + d] / pm;
  }
  if (extra) g += extra[i];
  dmass[i] = g;
}

// ---------------------------------------------------------------------------
// Structured-Gram matrix adjoint: one workgroup of D threads per matrix; the
// forward's vectors are recomputed in LDS, the D x D terms are swept by rows
// (thread d walks e) and by columns (thread e walks d).
template <int D>
struct StructBwdSmem {
  float sq[D], ms[D], var[D], dg[D], t[D], tc[D], hm[D], mhb[D];
  float dhm[D], dmhb[D], dt[D], dtc[D], ddg[D], dms[D];
  float red[D];
  float scal[8];
};

template <int D>
TAO_DEV float block_sum(float v, float* red) {
  const int tid = threadIdx.x;
  red[tid] = v;
  __syncthreads();
  float s = 0.0f;
  for (int i = 0; i < D; ++i) s += red[i];   // every thread, one order
  __syncthreads();
  return s;
}

template <int D>
__global__ __launch_bounds__(D) void structured_bwd_kernel(StructuredBwdParams p) {
  __shared__ StructBwdSmem<D> sm;
  const int mat = blockIdx.x, tid = threadIdx.x;
  const float n = p.count;
  const float* cr = p.cross + (size_t)mat * D * D;    // [d][e]
  const int blk = mat / (p.B * p.H), bh = mat % (p.B * p.H);
  const float* gt = p.dct + ((size_t)bh * p.dct_cap + blk) * D * D;   // dC^T: [e][d]
  const float sqd = p.square[(size_t)mat * D + tid];
  const float msd = p.mass[(size_t)mat * D + tid];
  const float pre = sqd - msd * msd / n;
  const float var = fmaxf(pre, 0.0f);
  sm.sq[tid] = sqd;
  sm.ms[tid] = msd;
  sm.var[tid] = var;
  const float vs = block_sum<D>(var, sm.red);
  const float ridge = block_sum<D>(sqd, sm.red) / (float)D;
  const bool zero = vs == 0.0f;
  const float dg = var + ridge;
  const float t = zero ? 0.0f : var / dg;
  sm.dg[tid] = dg;
  sm.t[tid] = t;
  const float ps = block_sum<D>(var * ridge / dg, sm.red);
  const float ss = zero ? 1.0f : ps;
  const float tm = block_sum<D>(t * msd, sm.red);
  const float hm = msd / dg + t * tm / ss;
  sm.hm[tid] = hm;
  __syncthreads();
  // column e = tid: tc[e] = sum_d t[d] cr[d][e]
  {
    float s = 0.0f;
    for (int d = 0; d < D; ++d) s += sm.t[d] * cr[(size_t)d * D + tid];
    sm.tc[tid] = s;
  }
  __syncthreads();
  // mhb[e] = sum_d ms[d] hb[d][e], hb = cr / dg + t tc / ss
  {
    const float tce = sm.tc[tid];
    float s = 0.0f;
    for (int d = 0; d < D; ++d)
      s += sm.ms[d] * (cr[(size_t)d * D + tid] / sm.dg[d] + sm.t[d] * tce / ss);
    sm.mhb[tid] = s;
  }
  const float den = n + block_sum<D>(msd * hm, sm.red);
  // dhm[d] = -sum_e G[d][e] mhb[e] / den (row d = tid; G[d][e] = gt[e][d])
  {
    float s = 0.0f;
    for (int e = 0; e < D; ++e) s += gt[(size_t)e * D + tid] * sm.mhb[e];
    sm.dhm[tid] = -s / den;
  }
  // dmhb[e] = -sum_d G[d][e] hm[d] / den (column e = tid)
  {
    float s = 0.0f;
    for (int d = 0; d < D; ++d) s += gt[(size_t)tid * D + d] * sm.hm[d];
    sm.dmhb[tid] = -s / den;
  }
  __syncthreads();
  const float dden = -block_sum<D>(sm.dhm[tid] * hm, sm.red) / den;
  float dms = dden * hm;
  float dhm = sm.dhm[tid] + dden * msd;
  // mhb: dms[d] += sum_e dmhb[e] hb[d][e]
  {
    float s = 0.0f;
    const float dgd = dg, td = t;
    for (int e = 0; e < D; ++e)
      s += sm.dmhb[e] * (cr[(size_t)tid * D + e] / dgd + td * sm.tc[e] / ss);
    dms += s;
  }
  // hm = ms / dg + t tm / ss
  dms += dhm / dg;
  float ddg = -dhm * msd / (dg * dg);
  float dt = dhm * tm / ss;
  const float dtm = block_sum<D>(dhm * t, sm.red) / ss;
  float dss = -tm * dtm / ss;
  // tm = sum t ms
  dt += dtm * msd;
  dms += dtm * t;
  // hb: dhb[d][e] = G[d][e] + ms[d] dmhb[e]; row sums for ddg and dt
  {
    float s_cr = 0.0f, s_tc = 0.0f;
    for (int e = 0; e < D; ++e) {
      const float dhb = gt[(size_t)e * D + tid] + msd * sm.dmhb[e];
      s_cr += dhb * cr[(size_t)tid * D + e];
      s_tc += dhb * sm.tc[e];
    }
    ddg -= s_cr / (dg * dg);
    dt += s_tc / ss;
  }
  // dtc[e] = sum_d dhb[d][e] t[d] / ss (column e = tid)
  {
    float s = 0.0f;
    const float dme = sm.dmhb[tid];
    for (int d = 0; d < D; ++d) s += (gt[(size_t)tid * D + d] + sm.ms[d] * dme) * sm.t[d];
    sm.dtc[tid] = s / ss;
  }
  __syncthreads();
  dss -= block_sum<D>(sm.dtc[tid] * sm.tc[tid], sm.red) / ss;
  // tc: dt[d] += sum_e dtc[e] cr[d][e]
  {
    float s = 0.0f;
    for (int e = 0; e < D; ++e) s += sm.dtc[e] * cr[(size_t)tid * D + e];
    dt += s;
  }
  // d cross[d][e] = dhb / dg + t[d] dtc[e] (row d = tid)
  {
    float* dcr = p.dcross + (size_t)mat * D * D + (size_t)tid * D;
    for (int e = 0; e < D; ++e) {
      const float dhb = gt[(size_t)e * D + tid] + msd * sm.dmhb[e];
      dcr[e] = dhb / dg + t * sm.dtc[e];
    }
  }
  // ss, ps, t, dg, ridge, var
  const float dps = zero ? 0.0f : dss;
  float dvar = dps * ridge / dg;
  const float dridge_ps = dps * block_sum<D>(var / dg, sm.red);
  ddg -= dps * var * ridge / (dg * dg);
  if (!zero) {
    dvar += dt / dg;
    ddg -= dt * var / (dg * dg);
  }
  dvar += ddg;
  const float dridge = dridge_ps + block_sum<D>(ddg, sm.red);
  float dsq = dridge / (float)D;
  if (pre >= 0.0f) {
    dsq += dvar;
    dms -= dvar * 2.0f * msd / n;
  }
  p.dsquare[(size_t)mat * D + tid] = dsq;
  p.dmass[(size_t)mat * D + tid] = dms;
}

__global__ __launch_bounds__(256) void square_diag_kernel(const float* dsq, float* s, int mats,
                                                          int D) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)mats * D * D;
  if (i >= total) return;
  const size_t mat = i / ((size_t)D * D);
  const int r = (int)(i / D % D), c = (int)(i % D);
  s[i] = r == c ? 2.0f * dsq[mat * D + r] : 0.0f;
}

__global__ __launch_bounds__(256) void page_add_kernel(float* fine, const float* page, int pages,
                                                       int group, int B, int H, int64_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t per = (size_t)B * H * n;
  const size_t total = (size_t)pages * group * per;
  if (i >= total) return;
  const size_t f = i / per, rest = i % per;
  fine[i] += page[(f / group) * per + rest];
}

}  // namespace

hipError_t launch_mix_bwd(const MixBwdParams& p, int head_dim, hipStream_t s) {
  if (p.n_items <= 0 || p.T <= 0) return hipSuccess;
  if (p.R < 1 || p.R > kMixMaxRank || p.ft % 32 || p.first_query % 32) return hipErrorInvalidValue;
  if (p.qsel && (p.n_items > kMixMaxItems || (p.n_items + 31) / 32 > p.qsel_words ||
                 p.qsel_words > 16))
    return hipErrorInvalidValue;
  if (!p.qsel && p.n_items > kMixMaxRank) return hipErrorInvalidValue;
  const int BH = p.B * p.H;
  const dim3 qgrid((unsigned)(((p.T + 31) / 32) * BH));
  const dim3 igrid((unsigned)(p.n_items * BH));
  if (head_dim == 128) {
    hipLaunchKernelGGL(mix_query_bwd_kernel<128>, qgrid, dim3(256), 0, s, p);
    hipLaunchKernelGGL(mix_item_bwd_kernel<128>, igrid, dim3(256), 0, s, p);
  } else if (head_dim == 64) {
    hipLaunchKernelGGL(mix_query_bwd_kernel<64>, qgrid, dim3(128), 0, s, p);
    hipLaunchKernelGGL(mix_item_bwd_kernel<64>, igrid, dim3(256), 0, s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_mass_grad(const float* dz, const float* dpz, const float* mass,
                            const float* extra, float* dmass, int fines, int pages, int group,
                            int B, int H, int head_dim, hipStream_t s) {
  const size_t total = (size_t)fines * B * H * head_dim;
  if (!total) return hipSuccess;
  if (pages > 0 && !dpz) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mass_grad_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     dz, dpz, mass, extra, dmass, fines, pages, group, B, H, head_dim);
  return hipGetLastError();
}

hipError_t launch_structured_bwd(const StructuredBwdParams& p, int head_dim, hipStream_t s) {
  if (p.count_mats <= 0) return hipSuccess;
  if (head_dim == 128)
    hipLaunchKernelGGL(structured_bwd_kernel<128>, dim3((unsigned)p.count_mats), dim3(128), 0, s,
                       p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(structured_bwd_kernel<64>, dim3((unsigned)p.count_mats), dim3(64), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_square_diag(const float* dsquare, float* s_, int mats, int head_dim,
                              hipStream_t st) {
  const size_t total = (size_t)mats * head_dim * head_dim;
  if (!total) return hipSuccess;
  hipLaunchKernelGGL(square_diag_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                     dsquare, s_, mats, head_dim);
  return hipGetLastError();
}

hipError_t launch_page_add(float* fine, const float* page, int pages, int group, int B, int H,
                           int64_t n, hipStream_t s) {
  const size_t total = (size_t)pages * group * B * H * n;
  if (!total) return hipSuccess;
  hipLaunchKernelGGL(page_add_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     fine, page, pages, group, B, H, n);
  return hipGetLastError();
}

}  // namespace tao
