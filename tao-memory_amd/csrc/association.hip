// Non-preset fine writers on gfx950: simplex-feature statistics, the
// regularised association solve, the structured (diagonal + rank-two)
// inverse, the chronological statistic sum and the feature-mass read
// coefficients.
//
// writer_stats_kernel (association_writer.py:11-18, structured_writer.py:5-13):
//   one 512-thread workgroup per (block n, head h). Tokens are taken 64 at a
//   time: 8 lanes per token form u = bf16(softmax_D(fp32 k)) (max and sum
//   over the 8 lanes' shuffles), u^T and v^T are staged in LDS, and
//   gram = u^T u, cross = u^T v run on v_mfma_f32_32x32x16_bf16 (m = d,
//   n = d' or e, k = token); u is bf16 and v is bf16, so every product is
//   exact and only the fp32 summation order differs from the reference's
//   matmul. mass = sum_t u and square_mass = sum_t u^2 are per-channel fp32
//   sums over the staged rows.
// association_solve_kernel (association_writer.py:21-32): one workgroup per
//   [D, D] pair, loaded in one round of float4 loads. The system
//   gram + (trace / D) I is factored in LDS by a blocked right-looking
//   Cholesky (16-column panels: the diagonal block by one wave in
//   registers, the rows below it one thread each, rank-16 trailing updates
//   on 4 x 4 register tiles), then cross is solved in place by forward and
//   back substitution, 16 rows a step with 4 x 4 tiles; C = bf16(X).
// structured_matrix_kernel (structured_writer.py:16-34): one workgroup per
//   pair; per-channel vectors and their sums in LDS, then thread e walks
//   column e of cross twice (hb and mass . hb, then the result).
// chrono_sum_kernel (association_writer.py:35-40): fp32 sum over the fine
//   axis in fine order.
// feature_coeff_kernel (association_writer.py:43-53): one wave per
//   (b, t, h); mass_p = sum_d h[d] exp(z_p[d]) by a wave reduction, then
//   out[p][d] = bf16(mass_p / sum_p mass_p * h[d]).
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

constexpr int kStatThreads = 512;
constexpr int kStatTokens = 64;

template <int D>
struct StatSmem {
  bf16_t ut[D][kStatTokens + 8];     // u^T [d][t]
  bf16_t vt[D][kStatTokens + 8];     // v^T [e][t]
};

// mode 0: gram + cross (+ mass when p.mass); mode 1: square_mass + cross + mass.
template <int D>
__global__ __launch_bounds__(kStatThreads) void writer_stats_kernel(WriterStatsParams p) {
  constexpr int DT = D / 32, KS = kStatTokens / 16, LPT = 8, CPL = D / LPT;
  __shared__ StatSmem<D> sm;
  const int n = blockIdx.x / p.H, h = blockIdx.x % p.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const bool structured = p.mode == 1;
  // output tiles: gram (mode 0 only) then cross; wave w owns tiles w, w + 8, ...
  const int n_tiles = (structured ? 1 : 2) * DT * DT;
  constexpr int TPW = (2 * DT * DT + 7) / 8;
  floatx16 acc[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[j][i] = 0.0f;
  float msum = 0.0f, ssum = 0.0f;          // thread tid < D: channel tid
  const int tk = tid / LPT, part = tid % LPT;
  // ring mode: block n = blk * B + b of a seal (see WriterStatsParams)
  const bool ring = p.starts != nullptr;
  int rb = 0, slot0 = 0;
  long long rel = 0;
  if (ring) {
    const long long start = p.starts[n / p.B];
    rb = n % p.B;
    rel = start - p.new_base;
    slot0 = (int)(start % p.L);
  }
  auto row_of = [&](const bf16_t* base, const int64_t* st, const bf16_t* ring_base, int t)
      __attribute__((always_inline)) -> const bf16_t* {
    if (!ring) return base + n * st[0] + (int64_t)t * st[1] + h * st[2];
    const long long r = rel + t;
    if (r >= 0) return base + rb * st[0] + r * st[1] + h * st[2];
    int slot = slot0 + t;
    slot = slot >= p.L ? slot - p.L : slot;
    return ring_base + (((size_t)rb * p.L + slot) * p.H + h) * D;
  };
  for (int t0 = 0; t0 < p.T; t0 += kStatTokens) {
    const int t = t0 + tk;
    float x[CPL];
    uint32_t vw[CPL / 2];
    if (t < p.T) {
      const bf16_t* kr = row_of(p.k, p.k_s, p.ring_raw, t) + part * CPL;
      const bf16_t* vr = row_of(p.v, p.v_s, p.ring_v, t) + part * CPL;
#pragma unroll
      for (int c = 0; c < CPL / 8; ++c) {
        const uint4 ku = *(const uint4*)(kr + 8 * c), vu = *(const uint4*)(vr + 8 * c);
        const uint32_t kw[4] = {ku.x, ku.y, ku.z, ku.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[8 * c + 2 * j] = __uint_as_float(kw[j] << 16);
          x[8 * c + 2 * j + 1] = __uint_as_float(kw[j] & 0xFFFF0000u);
        }
        vw[4 * c] = vu.x; vw[4 * c + 1] = vu.y; vw[4 * c + 2] = vu.z; vw[4 * c + 3] = vu.w;
      }
      float mx = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < CPL; ++j) mx = fmaxf(mx, x[j]);
#pragma unroll
      for (int off = 1; off < LPT; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      // u = r(e / s): e = correctly rounded fp32 exp(k - max); s = each
      // lane's CPL channels summed in channel order, then the 8 lanes'
      // partial sums pairwise (xor 1, 2, 4). Both orders are fixed so the
      // feature mass, and with it the descriptors that feed routing, are
      // bit-reproducible.
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) { x[j] = exp_cr(x[j] - mx); s += x[j]; }
#pragma unroll
      for (int off = 1; off < LPT; off <<= 1) s += __shfl_xor(s, off, 64);
#pragma unroll
      for (int j = 0; j < CPL; ++j) x[j] = rbf(x[j] / s);
    } else {
#pragma unroll
      for (int j = 0; j < CPL; ++j) x[j] = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL / 2; ++j) vw[j] = 0u;
    }
    __syncthreads();                      // previous chunk consumed
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int d = part * CPL + j;
      sm.ut[d][tk] = f2bf(x[j]);
      sm.vt[d][tk] = (bf16_t)((j & 1) ? (vw[j / 2] >> 16) : (vw[j / 2] & 0xFFFFu));
    }
    __syncthreads();
    if (tid < D && (p.mass || structured)) {
      const int cnt = min(kStatTokens, p.T - t0);
      for (int i = 0; i < cnt; ++i) {
        const float u = bf2f(sm.ut[tid][i]);
        msum += u;
        ssum = fmaf(u, u, ssum);
      }
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int tt = w + 8 * j;
      if (tt < n_tiles) {
        const bool is_cross = structured || tt >= DT * DT;
        const int r = structured ? tt : tt % (DT * DT);
        const int mt = r / DT, nt = r % DT;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bf16x8 a = as_bf16x8(*(const uint4*)&sm.ut[32 * mt + li][16 * ks + 8 * hl]);
          const bf16x8 b = is_cross
              ? as_bf16x8(*(const uint4*)&sm.vt[32 * nt + li][16 * ks + 8 * hl])
              : as_bf16x8(*(const uint4*)&sm.ut[32 * nt + li][16 * ks + 8 * hl]);
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
        }
      }
    }
  }
  const size_t mat = (size_t)n * p.H + h;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int tt = w + 8 * j;
    if (tt >= n_tiles) continue;
    const bool is_cross = structured || tt >= DT * DT;
    const int r = structured ? tt : tt % (DT * DT);
    const int mt = r / DT, nt = r % DT;
    float* out = (is_cross ? p.cross : p.gram) + mat * D * D;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 32 * mt + 8 * (i / 4) + 4 * hl + (i % 4);
      out[(size_t)row * D + 32 * nt + li] = acc[j][i];
    }
  }
  if (tid < D) {
    if (p.mass) p.mass[mat * D + tid] = msum;
    if (structured) p.gram[mat * D + tid] = ssum;   // square_mass
  }
}

constexpr int kSolveThreads = 1024;   // one workgroup per CU at D128 (135 KB LDS): 16 waves
constexpr int kSolvePanel = 16;       // Cholesky panel width and substitution block

template <int D>
struct SolveSmem {
  float a[D][D + 4];     // system, then its lower factor (rows 16-byte aligned)
  float x[D][D + 4];     // cross, then Y, then X
  float inv[D];          // reciprocal square roots of the pivots (1 / L[j][j])
  float red[kSolveThreads / 64];
};

TAO_DEV float read_lane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// acc[i] -= l[i] * r (componentwise), as one fp32 FMA per element.
TAO_DEV void sub_outer(float4 (&acc)[4], const float (&l)[4], const float4& r) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[i].x = fmaf(-l[i], r.x, acc[i].x);
    acc[i].y = fmaf(-l[i], r.y, acc[i].y);
    acc[i].z = fmaf(-l[i], r.z, acc[i].z);
    acc[i].w = fmaf(-l[i], r.w, acc[i].w);
  }
}

template <int D>
__global__ __launch_bounds__(kSolveThreads) void association_solve_kernel(AssocSolveParams p) {
  extern __shared__ __align__(16) unsigned char solve_smem[];
  SolveSmem<D>& sm = *reinterpret_cast<SolveSmem<D>*>(solve_smem);
  const int mat = blockIdx.x;
  const int tid = threadIdx.x;
  const int blk = (p.to_slots || p.rhs_t) ? mat / (p.B * p.H) : 0;
  if (p.to_slots == 2 && (p.fine_first + blk) % p.group != p.group - 1) return;   // uniform
  const float* g = p.gram + (size_t)mat * D * D;
  const float* c = p.cross + (size_t)mat * D * D;
  const float* rt = nullptr;   // transposed right-hand side ([e][d])
  if (p.rhs_t) {
    const int b = (mat / p.H) % p.B, h = mat % p.H;
    rt = p.rhs_t + (((size_t)b * p.H + h) * p.rhs_cap + blk) * D * D;
  }
  // Every load of the system in one round: the diagonal (for the ridge),
  // then gram and the right-hand side as float4 (rows of D floats).
  constexpr int V4 = D * D / 4 / kSolveThreads;   // float4 per thread and matrix
  static_assert(D * D % (4 * kSolveThreads) == 0, "whole float4 per thread");
  const float gd = tid < D ? g[(size_t)tid * D + tid] : 0.0f;
  float4 gv[V4], cv[V4];
#pragma unroll
  for (int k = 0; k < V4; ++k) {
    const int i4 = tid + k * kSolveThreads;
    gv[k] = ((const float4*)g)[i4];
    cv[k] = ((const float4*)(rt ? rt : c))[i4];
  }
#pragma unroll
  for (int k = 0; k < V4; ++k) {
    const int i = 4 * (tid + k * kSolveThreads), r = i / D, col = i % D;
    *(float4*)&sm.a[r][col] = gv[k];
    if (rt) {   // rt[e][d] with e = r, d = col .. col + 3: x[d][e]
      sm.x[col][r] = cv[k].x;
      sm.x[col + 1][r] = cv[k].y;
      sm.x[col + 2][r] = cv[k].z;
      sm.x[col + 3][r] = cv[k].w;
    } else {
      *(float4*)&sm.x[r][col] = cv[k];
    }
  }
  // ridge = trace / D, added to the staged diagonal
  const float tr = wave_sum_fold(gd);
  if ((tid & 63) == 0) sm.red[tid >> 6] = tr;
  __syncthreads();
  float trace = 0.0f;
#pragma unroll
  for (int i = 0; i < kSolveThreads / 64; ++i) trace += sm.red[i];
  const float ridge = trace / (float)D;
  if (tid < D) sm.a[tid][tid] = gd + ridge;
  // Blocked right-looking Cholesky, PB columns a step. Wave 0 factors the
  // panel's PB x PB diagonal block in registers (lane l holds row jb + l;
  // the pivot and the multipliers L[jb + c2][j] come from their lanes by
  // readlane); then thread t solves row jb + PB + t of the panel against
  // it, column by column; then every thread applies the rank-PB update to
  // 4 x 4 tiles of the trailing lower triangle from float4 rows (the upper
  // triangle is never read, so diagonal tiles are updated whole). Each
  // element sees the operations of the unblocked factorization in the same
  // order: one fp32 FMA per earlier column, in column order, then the
  // scaling by its column's pivot. Pivots are taken by v_rsq_f32 (about
  // 1 ulp): L[j][j] = pivot * rsq(pivot), and every division by L[j][j],
  // here and in the substitutions, is a product with rsq(pivot) (kept in
  // sm.inv); these ulp-level differences sit far below the bf16 rounding of
  // the result.
  constexpr int PB = kSolvePanel;
  static_assert(D % PB == 0 && PB <= 64, "panel layout");
  int bad = 0;
  const int lane = tid & 63;
  for (int jb = 0; jb < D; jb += PB) {
    __syncthreads();
    if (tid < 64) {
      float pr[PB];
      const int rowk = jb + lane;
#pragma unroll
      for (int c = 0; c < PB; ++c) pr[c] = lane < PB ? sm.a[rowk][jb + c] : 0.0f;
#pragma unroll
      for (int c = 0; c < PB; ++c) {
        const int j = jb + c;
        const float piv = read_lane(pr[c], c);           // row j: lane c
        if (!(piv > 0.0f)) bad = bad ? bad : j + 1;
        const float rj = __builtin_amdgcn_rsqf(piv);
        if (lane > c) pr[c] = pr[c] * rj;
        if (lane == c) pr[c] = piv * rj;
        if (lane == 0) sm.inv[j] = rj;
#pragma unroll
        for (int c2 = c + 1; c2 < PB; ++c2) {
          const float f = read_lane(pr[c], c2);          // L[jb + c2][j]
          if (lane >= c2) pr[c2] = fmaf(-pr[c], f, pr[c2]);
        }
      }
      if (lane < PB) {
#pragma unroll
        for (int c = 0; c < PB; ++c)
          if (c <= lane) sm.a[rowk][jb + c] = pr[c];
      }
    }
    __syncthreads();
    if (tid < D - jb - PB) {
      const int rowk = jb + PB + tid;
      float l[PB];
#pragma unroll
      for (int q = 0; q < PB / 4; ++q) {
        const float4 v = *(const float4*)&sm.a[rowk][jb + 4 * q];
        l[4 * q] = v.x; l[4 * q + 1] = v.y; l[4 * q + 2] = v.z; l[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int c = 0; c < PB; ++c) {
        float v = l[c];
#pragma unroll
        for (int u = 0; u < c; ++u) v = fmaf(-l[u], sm.a[jb + c][jb + u], v);
        l[c] = v * sm.inv[jb + c];
      }
#pragma unroll
      for (int q = 0; q < PB / 4; ++q)
        *(float4*)&sm.a[rowk][jb + 4 * q] = make_float4(l[4 * q], l[4 * q + 1], l[4 * q + 2],
                                                        l[4 * q + 3]);
    }
    __syncthreads();
    const int r0 = jb + PB, nt = (D - r0) / 4;
    for (int t = tid; t < nt * (nt + 1) / 2; t += kSolveThreads) {
      int kt = (int)((__builtin_sqrtf(8.0f * (float)t + 1.0f) - 1.0f) * 0.5f);
      while (kt * (kt + 1) / 2 > t) --kt;
      while ((kt + 1) * (kt + 2) / 2 <= t) ++kt;
      const int ct = t - kt * (kt + 1) / 2;
      const int k0 = r0 + 4 * kt, c0 = r0 + 4 * ct;
      float4 acc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = *(const float4*)&sm.a[k0 + i][c0];
#pragma unroll
      for (int q = 0; q < PB / 4; ++q) {
        float4 lk[4], lc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lk[i] = *(const float4*)&sm.a[k0 + i][jb + 4 * q];
          lc[i] = *(const float4*)&sm.a[c0 + i][jb + 4 * q];
        }
        // column jb + 4q + s: acc[i][j] -= L[k0 + i][.] * L[c0 + j][.]
        const float lks[4][4] = {{lk[0].x, lk[1].x, lk[2].x, lk[3].x},
                                 {lk[0].y, lk[1].y, lk[2].y, lk[3].y},
                                 {lk[0].z, lk[1].z, lk[2].z, lk[3].z},
                                 {lk[0].w, lk[1].w, lk[2].w, lk[3].w}};
        const float4 lcs[4] = {make_float4(lc[0].x, lc[1].x, lc[2].x, lc[3].x),
                               make_float4(lc[0].y, lc[1].y, lc[2].y, lc[3].y),
                               make_float4(lc[0].z, lc[1].z, lc[2].z, lc[3].z),
                               make_float4(lc[0].w, lc[1].w, lc[2].w, lc[3].w)};
#pragma unroll
        for (int sidx = 0; sidx < 4; ++sidx) sub_outer(acc, lks[sidx], lcs[sidx]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) *(float4*)&sm.a[k0 + i][c0] = acc[i];
    }
  }
  __syncthreads();
  if (p.info && tid == 0) p.info[mat] = bad;
  // Forward (L Y = X) then back (L^T X = Y) substitution, PB rows a step:
  // thread e solves the step's rows of column e, then every thread removes
  // them from a 4 x 4 tile of the remaining rows (one FMA per solved row, in
  // row order); two barriers a step.
  constexpr int NCT = D / 4;
  for (int ib = 0; ib < D; ib += PB) {
    if (tid < D) {
      const int e = tid;
      float y[PB];
#pragma unroll
      for (int t = 0; t < PB; ++t) {
        float v = sm.x[ib + t][e];
#pragma unroll
        for (int u = 0; u < t; ++u) v = fmaf(-sm.a[ib + t][ib + u], y[u], v);
        y[t] = v * sm.inv[ib + t];
        sm.x[ib + t][e] = y[t];
      }
    }
    __syncthreads();
    const int r0 = ib + PB;
    for (int t = tid; t < (D - r0) / 4 * NCT; t += kSolveThreads) {
      const int k0 = r0 + 4 * (t / NCT), e0 = 4 * (t % NCT);
      float4 acc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = *(const float4*)&sm.x[k0 + i][e0];
#pragma unroll
      for (int q = 0; q < PB / 4; ++q) {
        float4 lk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) lk[i] = *(const float4*)&sm.a[k0 + i][ib + 4 * q];
        const float lks[4][4] = {{lk[0].x, lk[1].x, lk[2].x, lk[3].x},
                                 {lk[0].y, lk[1].y, lk[2].y, lk[3].y},
                                 {lk[0].z, lk[1].z, lk[2].z, lk[3].z},
                                 {lk[0].w, lk[1].w, lk[2].w, lk[3].w}};
#pragma unroll
        for (int sidx = 0; sidx < 4; ++sidx)
          sub_outer(acc, lks[sidx], *(const float4*)&sm.x[ib + 4 * q + sidx][e0]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) *(float4*)&sm.x[k0 + i][e0] = acc[i];
    }
    __syncthreads();
  }
  for (int ib = D - PB; ib >= 0; ib -= PB) {
    if (tid < D) {
      const int e = tid;
      float xv[PB];
#pragma unroll
      for (int t = PB - 1; t >= 0; --t) {
        float v = sm.x[ib + t][e];
#pragma unroll
        for (int u = t + 1; u < PB; ++u) v = fmaf(-sm.a[ib + u][ib + t], xv[u], v);
        xv[t] = v * sm.inv[ib + t];
        sm.x[ib + t][e] = xv[t];
      }
    }
    __syncthreads();
    for (int t = tid; t < ib / 4 * NCT; t += kSolveThreads) {
      const int k0 = 4 * (t / NCT), e0 = 4 * (t % NCT);
      float4 acc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = *(const float4*)&sm.x[k0 + i][e0];
#pragma unroll
      for (int t2 = 0; t2 < PB; ++t2) {
        // row ib + t2 of L, columns k0 .. k0 + 3 (L^T[k][ib + t2])
        const float4 lr = *(const float4*)&sm.a[ib + t2][k0];
        const float l4[4] = {lr.x, lr.y, lr.z, lr.w};
        sub_outer(acc, l4, *(const float4*)&sm.x[ib + t2][e0]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) *(float4*)&sm.x[k0 + i][e0] = acc[i];
    }
    __syncthreads();
  }
  if (p.out_f32) {
    float* out = p.out_f32 + (size_t)mat * D * D;
    for (int i = tid; i < D * D; i += kSolveThreads) out[i] = sm.x[i / D][i % D];
    return;
  }
  if (!p.to_slots) {
    bf16_t* out = p.out + (size_t)mat * D * D;
    for (int i = tid; i < D * D; i += kSolveThreads) out[i] = f2bf(sm.x[i / D][i % D]);
    return;
  }
  // C^T into a bank (fine) or page slot: dst[e][d] = X[d][e]
  const int b = (mat / p.H) % p.B, h = mat % p.H;
  const int slot = p.to_slots == 1 ? p.first_slot + blk : (p.fine_first + blk) / p.group;
  bf16_t* dst = p.out + (((size_t)b * p.H + h) * p.cap + slot) * D * D;
  for (int i = tid; i < D * D; i += kSolveThreads) dst[i] = f2bf(sm.x[i % D][i / D]);
}

template <int D>
__global__ __launch_bounds__(D) void structured_matrix_kernel(StructuredParams p) {
  __shared__ float diag[D], tv[D], mv[D], hmv[D], red[4][D / 64 > 0 ? D / 64 : 1];
  const int mat = blockIdx.x, d = threadIdx.x;
  if (p.to_slots == 2 && (p.first_slot + mat / (p.B * p.H)) % p.group != p.group - 1)
    return;   // uniform: only blocks that complete a page
  const float count = p.count;
  const float sq = p.square[(size_t)mat * D + d];
  const float ms = p.mass[(size_t)mat * D + d];
  const float variance = fmaxf(sq - ms * ms / count, 0.0f);
  // four block sums: variance, square_mass, then (after the ridge) the
  // positive sum and t . mass
  auto block_sum = [&](float v, int slot) __attribute__((always_inline)) {
    v = wave_sum_fold(v);
    if ((d & 63) == 0) red[slot][d >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < D / 64; ++i) s += red[slot][i];
    return s;
  };
  const float variance_sum = block_sum(variance, 0);
  const float ridge = block_sum(sq, 1) / (float)D;
  const float diagonal = variance + ridge;
  const bool zero = variance_sum == 0.0f;
  const float t = zero ? 0.0f : variance / diagonal;
  const float positive_sum = block_sum(variance * ridge / diagonal, 2);
  const float safe_sum = zero ? 1.0f : positive_sum;
  const float tmass = block_sum(t * ms, 3);
  const float hm = ms / diagonal + t * tmass / safe_sum;
  diag[d] = diagonal; tv[d] = t; mv[d] = ms; hmv[d] = hm;
  __syncthreads();
  float mhm = 0.0f;
  for (int i = 0; i < D; ++i) mhm = fmaf(mv[i], hmv[i], mhm);
  const float denominator = count + mhm;
  // thread e: column e of cross
  const int e = d;
  const float* cr = p.cross + (size_t)mat * D * D;
  float t_cross = 0.0f;
  for (int i = 0; i < D; ++i) t_cross = fmaf(tv[i], cr[(size_t)i * D + e], t_cross);
  float mass_hb = 0.0f;
  for (int i = 0; i < D; ++i) {
    const float hb = cr[(size_t)i * D + e] / diag[i] + tv[i] * t_cross / safe_sum;
    mass_hb = fmaf(mv[i], hb, mass_hb);
  }
  if (p.to_slots) {
    // C^T into the fine bank: row e of slot first_slot + blk (1), or of the
    // page that fine slot completes (2).
    const int blk = mat / (p.B * p.H), b = mat / p.H % p.B, h = mat % p.H;
    const int slot = p.to_slots == 1 ? p.first_slot + blk : (p.first_slot + blk) / p.group;
    bf16_t* out = p.out + ((((size_t)b * p.H + h) * p.cap + slot) * D + e) * D;
    for (int i = 0; i < D; ++i) {
      const float hb = cr[(size_t)i * D + e] / diag[i] + tv[i] * t_cross / safe_sum;
      out[i] = f2bf(hb - hmv[i] * mass_hb / denominator);
    }
    return;
  }
  bf16_t* out = p.out + (size_t)mat * D * D;
  for (int i = 0; i < D; ++i) {
    const float hb = cr[(size_t)i * D + e] / diag[i] + tv[i] * t_cross / safe_sum;
    out[(size_t)i * D + e] = f2bf(hb - hmv[i] * mass_hb / denominator);
  }
}

// One thread per (batch, head, channel), the seal blocks in seal order: the
// fine's z = r(log mass) from its own mass, and fine_mass[slot] = the run's
// fp32 total through this fine, run + mass (tao_stream.py:463-467). A run
// starts at fine 0 and, with page_runs, at every page's first fine; so
// r(log fine_mass[last fine]) is the page (or pending) descriptor
// (tao_stream.py:280-283, 483). The streaming index-only state never
// restarts its run, as the reference clears pending_mass only when it
// builds page values (:488-497); the full-sequence path sums per page
// (:543-549).
template <int D>
__global__ __launch_bounds__(256) void feature_desc_kernel(FeatureDescParams p) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)p.B * p.H * D) return;
  const int d = (int)(i % D);
  const int64_t bh = i / D;
  const size_t row = (size_t)bh * p.cap * D + d;
  float run = p.first_slot > 0 ? p.fine_mass[row + (size_t)(p.first_slot - 1) * D] : 0.0f;
  for (int blk = 0; blk < p.count; ++blk) {
    const int slot = p.first_slot + blk;
    const float m = p.mass[((size_t)blk * p.B * p.H + bh) * D + d];
    const bool fresh = p.page_runs ? slot % p.group == 0 : slot == 0;
    run = fresh ? m : run + m;
    p.fine_z[row + (size_t)slot * D] = f2bf(log_bf(m));
    p.fine_mass[row + (size_t)slot * D] = run;
  }
}

__global__ __launch_bounds__(256) void chrono_sum_kernel(const float* x, float* out, int64_t outer,
                                                          int fines, int64_t inner) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= outer * inner) return;
  const int64_t o = i / inner, r = i % inner;
  const float* base = x + o * fines * inner + r;
  float s = base[0];
  for (int f = 1; f < fines; ++f) s += base[(int64_t)f * inner];
  out[i] = s;
}

template <int D>
__global__ __launch_bounds__(256) void feature_coeff_kernel(FeatureCoeffParams p) {
  constexpr int PL = D / 64;             // channels per lane
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= p.B * p.T * p.H) return;   // wave-uniform
  const int h = row % p.H, t = (row / p.H) % p.T, b = row / (p.H * p.T);
  const bf16_t* hr = p.h + b * p.h_s[0] + (int64_t)t * p.h_s[1] + h * p.h_s[2];
  const bf16_t* zr = p.z + b * p.z_s[0] + (int64_t)t * p.z_s[1] + h * p.z_s[2];
  float hv[PL];
#pragma unroll
  for (int j = 0; j < PL; ++j) hv[j] = bf2f(hr[lane + 64 * j]);
  auto mass_of = [&](int pg) __attribute__((always_inline)) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < PL; ++j) s = fmaf(hv[j], __expf(bf2f(zr[pg * p.z_s[3] + lane + 64 * j])), s);
    return wave_sum_fold(s);
  };
  float total = 0.0f;
  for (int pg = 0; pg < p.P; ++pg) total += mass_of(pg);
  bf16_t* out = p.out + (size_t)row * p.P * D;
  for (int pg = 0; pg < p.P; ++pg) {
    const float mix = mass_of(pg) / total;
#pragma unroll
    for (int j = 0; j < PL; ++j) out[(size_t)pg * D + lane + 64 * j] = f2bf(mix * hv[j]);
  }
}

__global__ __launch_bounds__(256) void assoc_pending_kernel(AssocPendingParams p, int dd) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per = (int64_t)p.B * p.H * dd;
  if (i >= per) return;
  const int64_t bh = i / dd, e = i % dd;                // bh = b * H + h
  const bool two = p.cross != nullptr;                  // a second statistic summed alike
  float pg = p.pending_gram[i], pc = two ? p.pending_cross[i] : 0.0f;
  for (int blk = 0; blk < p.count; ++blk) {
    const int slot = p.first_slot + blk;
    const int64_t at = ((int64_t)blk * p.B * p.H + bh) * dd + e;   // (blk, b, h) = blk * B * H + bh
    const bool fresh = p.reset_pages ? slot % p.group == 0 : slot == 0;
    pg = fresh ? p.gram[at] : pg + p.gram[at];
    if (two) pc = fresh ? p.cross[at] : pc + p.cross[at];
    if (p.reset_pages && slot % p.group == p.group - 1) {
      p.gram[at] = pg;
      if (two) p.cross[at] = pc;
    }
  }
  p.pending_gram[i] = pg;
  if (two) p.pending_cross[i] = pc;
}

}  // namespace

hipError_t launch_assoc_pending(const AssocPendingParams& p, int head_dim, hipStream_t s) {
  return launch_pending_sums(p, head_dim * head_dim, s);
}

hipError_t launch_pending_sums(const AssocPendingParams& p, int dd, hipStream_t s) {
  const int64_t n = (int64_t)p.B * p.H * dd;
  if (n <= 0 || p.count <= 0) return hipSuccess;
  hipLaunchKernelGGL(assoc_pending_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p,
                     dd);
  return hipGetLastError();
}

hipError_t launch_writer_stats(const WriterStatsParams& p, int head_dim, hipStream_t s) {
  const dim3 grid((unsigned)(p.N * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(writer_stats_kernel<128>, grid, dim3(kStatThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(writer_stats_kernel<64>, grid, dim3(kStatThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_association_solve(const AssocSolveParams& p, int head_dim, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  if (head_dim == 128) {
    constexpr size_t bytes = sizeof(SolveSmem<128>);
    static bool attr = false;
    if (!attr) {
      const hipError_t e = hipFuncSetAttribute((const void*)association_solve_kernel<128>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)bytes);
      if (e != hipSuccess) return e;
      attr = true;
    }
    hipLaunchKernelGGL(association_solve_kernel<128>, dim3((unsigned)p.count),
                       dim3(kSolveThreads), bytes, s, p);
  } else if (head_dim == 64) {
    hipLaunchKernelGGL(association_solve_kernel<64>, dim3((unsigned)p.count),
                       dim3(kSolveThreads), sizeof(SolveSmem<64>), s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_structured_matrix(const StructuredParams& p, int head_dim, hipStream_t s) {
  if (p.count_mats <= 0) return hipSuccess;
  if (head_dim == 128)
    hipLaunchKernelGGL(structured_matrix_kernel<128>, dim3((unsigned)p.count_mats), dim3(128), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(structured_matrix_kernel<64>, dim3((unsigned)p.count_mats), dim3(64), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_feature_descriptors(const FeatureDescParams& p, int head_dim, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  const int64_t n = (int64_t)p.B * p.H * head_dim;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (head_dim == 128)
    hipLaunchKernelGGL(feature_desc_kernel<128>, grid, dim3(256), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(feature_desc_kernel<64>, grid, dim3(256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---- regularized writer backward (see AssocBwdParams)

__global__ __launch_bounds__(256) void block_starts_kernel(int64_t* starts, int count,
                                                            int64_t step) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < count) starts[i] = (int64_t)i * step;
}

// One workgroup per matrix: S[i][j] = -(W Y^T + Y W^T)[i][j] + 2 tr(-W Y^T) / D
// [i == j], with W and Y staged in LDS (rows padded by one float). Thread
// entries run i fastest (distinct banks for W[i][.], Y[i][.]); S is
// symmetric, so entry (i, j) is stored at [j][i] for coalesced stores.
template <int D>
struct GramBwdSmem {
  float w[D][D + 1];
  float y[D][D + 1];
  float red[4];
};

template <int D>
__global__ __launch_bounds__(256) void assoc_gram_bwd_kernel(AssocBwdParams p) {
  extern __shared__ __align__(16) unsigned char gram_bwd_smem[];
  GramBwdSmem<D>& sm = *reinterpret_cast<GramBwdSmem<D>*>(gram_bwd_smem);
  const int mat = blockIdx.x, tid = threadIdx.x;
  const float* w = p.w + (size_t)mat * D * D;
  const float* y = p.y + (size_t)mat * D * D;
  float tr = 0.0f;
  for (int i = tid; i < D * D; i += 256) {
    const float wv = w[i], yv = y[i];
    sm.w[i / D][i % D] = wv;
    sm.y[i / D][i % D] = yv;
    tr += wv * yv;
  }
  tr = wave_sum_fold(tr);
  if ((tid & 63) == 0) sm.red[tid >> 6] = tr;
  __syncthreads();
  const float trace = -(sm.red[0] + sm.red[1] + sm.red[2] + sm.red[3]);   // tr(-W Y^T)
  float* out = p.s + (size_t)mat * D * D;
  for (int idx = tid; idx < D * D; idx += 256) {
    const int i = idx % D, j = idx / D;
    float acc = 0.0f;
    for (int e = 0; e < D; ++e) acc += sm.w[i][e] * sm.y[j][e] + sm.y[i][e] * sm.w[j][e];
    out[(size_t)j * D + i] = -acc + (i == j ? 2.0f * trace / (float)D : 0.0f);
  }
}

// One workgroup per (fine block, batch, head), 8 waves x 32 tokens. Lane
// (li, hl) of wave w holds token 32 w + li's channels 16 kk + 8 hl + j in
// the MFMA A layout: u = r(softmax_D(raw_k)) and v. du = V W^T + U S (B
// operand column d: row d of W, of S); dv += U W (column e: row e of W^T).
template <int D>
struct BlockBwdSmem {
  bf16_t w[D][D + 8];    // W [d][e]
  bf16_t wt[D][D + 8];   // W^T [e][d]
  bf16_t sg[D][D + 8];   // S [d][d']
  float mx[256], iz[256];   // per token: max and 1 / sum of exp
};

template <int D>
__global__ __launch_bounds__(512) void assoc_block_bwd_kernel(AssocBwdParams p) {
  constexpr int KK = D / 16, DT = D / 32;
  extern __shared__ __align__(16) unsigned char block_bwd_smem[];
  BlockBwdSmem<D>& sm = *reinterpret_cast<BlockBwdSmem<D>*>(block_bwd_smem);
  const int mat = blockIdx.x;
  const int f = mat / (p.B * p.H), b = (mat / p.H) % p.B, h = mat % p.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const float* wg = p.w + (size_t)mat * D * D;
  const float* sg = p.s + (size_t)mat * D * D;
  for (int i = tid; i < D * D; i += 512) {
    const int r = i / D, c = i % D;
    const bf16_t wv = f2bf(wg[i]);
    sm.w[r][c] = wv;
    sm.wt[c][r] = wv;
    sm.sg[r][c] = f2bf(sg[i]);
  }
  const int tok0 = f * p.ft;
  const int t_row = tok0 + 32 * w + li;
  const bf16_t* krow = p.raw_k.p + b * p.raw_k.sb + (int64_t)t_row * p.raw_k.st + h * p.raw_k.sh;
  const bf16_t* vrow = p.v.p + b * p.v.sb + (int64_t)t_row * p.v.st + h * p.v.sh;
  // softmax over the channels of this lane's token (both halves of the row)
  float kv[KK][8];
  float m = -__builtin_inff();
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    const uint4 ku = *(const uint4*)(krow + 16 * kk + 8 * hl);
    const uint32_t kw[4] = {ku.x, ku.y, ku.z, ku.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kv[kk][2 * j] = __uint_as_float(kw[j] << 16);
      kv[kk][2 * j + 1] = __uint_as_float(kw[j] & 0xFFFF0000u);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, kv[kk][j]);
  }
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float z = 0.0f;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
#pragma unroll
    for (int j = 0; j < 8; ++j) { kv[kk][j] = __expf(kv[kk][j] - m); z += kv[kk][j]; }
  z += __shfl_xor(z, 32, 64);
  const float iz = 1.0f / z;
  if (hl == 0) { sm.mx[32 * w + li] = m; sm.iz[32 * w + li] = iz; }
  bf16x8 ua[KK], va[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    va[kk] = as_bf16x8(*(const uint4*)(vrow + 16 * kk + 8 * hl));
    uint32_t pk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) pk[j] = pack_bf16x2(kv[kk][2 * j] * iz, kv[kk][2 * j + 1] * iz);
    ua[kk] = as_bf16x8(make_uint4(pk[0], pk[1], pk[2], pk[3]));
  }
  __syncthreads();
  // du tiles (lane = column d = 32 t + li, rows = tokens 8 (i/4) + 4 hl + i%4)
  floatx16 du[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) du[t][i] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      du[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          va[kk], as_bf16x8(*(const uint4*)&sm.w[32 * t + li][16 * kk + 8 * hl]), du[t], 0, 0, 0);
      du[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          ua[kk], as_bf16x8(*(const uint4*)&sm.sg[32 * t + li][16 * kk + 8 * hl]), du[t], 0, 0, 0);
    }
  }
  // Feature writers: d of the block's mass sum_t u_t reaches every token's u.
  if (p.dmass) {
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const float dm = p.dmass[(size_t)mat * D + 32 * t + li];
#pragma unroll
      for (int i = 0; i < 16; ++i) du[t][i] += dm;
    }
  }
  // p at the accumulator positions, and sum_d p du per token row
  float pv[DT][16], part[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) part[i] = 0.0f;
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const int d = 32 * t + li;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = 32 * w + 8 * (i / 4) + 4 * hl + (i % 4);
      const float kx = bf2f(p.raw_k.p[b * p.raw_k.sb + (int64_t)(tok0 + r) * p.raw_k.st +
                                      h * p.raw_k.sh + d]);
      pv[t][i] = __expf(kx - sm.mx[r]) * sm.iz[r];
      part[i] += pv[t][i] * du[t][i];
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) part[i] += __shfl_xor(part[i], off, 64);
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const int d = 32 * t + li;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = tok0 + 32 * w + 8 * (i / 4) + 4 * hl + (i % 4);
      p.dk[(((size_t)b * p.T + tok) * p.H + h) * D + d] = pv[t][i] * (du[t][i] - part[i]);
    }
  }
  // dv += U W (lane = column e)
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          ua[kk], as_bf16x8(*(const uint4*)&sm.wt[32 * t + li][16 * kk + 8 * hl]), acc, 0, 0, 0);
    const int e = 32 * t + li;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = tok0 + 32 * w + 8 * (i / 4) + 4 * hl + (i % 4);
      p.dv[(((size_t)b * p.T + tok) * p.H + h) * D + e] += acc[i];
    }
  }
}

__global__ __launch_bounds__(256) void page_sum_kernel(const float* x, float* out, int pages,
                                                        int group, int B, int H, int64_t dd) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per = (int64_t)B * H * dd;
  if (i >= (int64_t)pages * per) return;
  const int64_t g = i / per, r = i % per;               // r = (b H + h) dd + e
  float acc = x[(g * group) * per + r];
  for (int k = 1; k < group; ++k) acc += x[(g * group + k) * per + r];
  out[i] = acc;
}

__global__ __launch_bounds__(256) void page_to_fines_kernel(float* w, float* s, const float* wp,
                                                            const float* sp, int fines, int group,
                                                            int B, int H, int64_t dd) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per = (int64_t)B * H * dd;
  const int full = (fines / group) * group;             // fines of completed pages
  if (i >= (int64_t)full * per) return;
  const int64_t f = i / per, r = i % per;
  const int64_t at = (f / group) * per + r;
  w[i] += wp[at];
  s[i] += sp[at];
}

hipError_t launch_page_sum(const float* x, float* out, int pages, int group, int B, int H,
                           int64_t dd, hipStream_t s) {
  const int64_t n = (int64_t)pages * B * H * dd;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(page_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, out,
                     pages, group, B, H, dd);
  return hipGetLastError();
}

hipError_t launch_page_to_fines(float* w, float* s_, const float* wp, const float* sp, int fines,
                                int group, int B, int H, int64_t dd, hipStream_t s) {
  const int64_t n = (int64_t)((fines / group) * group) * B * H * dd;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(page_to_fines_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w,
                     s_, wp, sp, fines, group, B, H, dd);
  return hipGetLastError();
}

hipError_t launch_block_starts(int64_t* starts, int count, int64_t step, hipStream_t s) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(block_starts_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s,
                     starts, count, step);
  return hipGetLastError();
}

template <typename K>
hipError_t big_lds(K kernel, size_t bytes) {
  return hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)bytes);
}

hipError_t launch_assoc_gram_bwd(const AssocBwdParams& p, int head_dim, hipStream_t s) {
  if (p.mats <= 0) return hipSuccess;
  if (head_dim == 128) {
    const size_t bytes = sizeof(GramBwdSmem<128>);
    hipError_t e = big_lds(assoc_gram_bwd_kernel<128>, bytes);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(assoc_gram_bwd_kernel<128>, dim3((unsigned)p.mats), dim3(256), bytes, s, p);
  } else if (head_dim == 64) {
    hipLaunchKernelGGL(assoc_gram_bwd_kernel<64>, dim3((unsigned)p.mats), dim3(256),
                       sizeof(GramBwdSmem<64>), s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_assoc_block_bwd(const AssocBwdParams& p, int head_dim, hipStream_t s) {
  if (p.mats <= 0) return hipSuccess;
  if (p.ft != 256) return hipErrorInvalidValue;
  if (head_dim == 128) {
    const size_t bytes = sizeof(BlockBwdSmem<128>);
    hipError_t e = big_lds(assoc_block_bwd_kernel<128>, bytes);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(assoc_block_bwd_kernel<128>, dim3((unsigned)p.mats), dim3(512), bytes, s, p);
  } else if (head_dim == 64) {
    hipLaunchKernelGGL(assoc_block_bwd_kernel<64>, dim3((unsigned)p.mats), dim3(512),
                       sizeof(BlockBwdSmem<64>), s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_chrono_sum(const float* x, float* out, int64_t outer, int fines, int64_t inner,
                             hipStream_t s) {
  const int64_t n = outer * inner;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(chrono_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, out,
                     outer, fines, inner);
  return hipGetLastError();
}

hipError_t launch_feature_coeff(const FeatureCoeffParams& p, int head_dim, hipStream_t s) {
  const int64_t rows = (int64_t)p.B * p.T * p.H;
  if (rows <= 0 || p.P <= 0) return hipSuccess;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (head_dim == 128)
    hipLaunchKernelGGL(feature_coeff_kernel<128>, grid, dim3(256), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(feature_coeff_kernel<64>, grid, dim3(256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace tao
