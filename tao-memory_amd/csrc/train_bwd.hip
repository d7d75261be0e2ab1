// Backward of the full-sequence read (tao_attention, operator.py:40-52) for
// gfx950: the adjoints the reference takes by autograd through
// _fuse_training (operator.py:21-38), the local SDPA of
// _local_training_corrected_4k (tao_stream.py:760-787), the selected read
// (selected_read.py:175-187), the page / segment softmaxes and logsumexps
// (tao_stream.py:530-665) and the softmax writer (tao_stream.py:80-123).
//
// Gradients are those of the forward's function at the forward's values and
// selections (the selection has no derivative, tao_stream.py:647-650);
// accumulation is fp32 throughout, MFMA operands are bf16.
#include <algorithm>

#include "tao_launch.h"
#include "tao_common.h"
#include "tao_fusion.h"

namespace tao {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

TAO_DEV bf16x8 as_bf16x8(const uint4& u) {
  bf16x8 r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

// ---------------------------------------------------------------------------
// Fusion adjoint (operator.py:21-38). Workgroup = (64-token chunk of one
// batch row, head); thread (e = tid % D, lane row r = tid / D) walks the
// chunk's tokens r, r + 256 / D, ... Per element, with the forward's bf16
// scores s_i and branch values x = (2 local, gain coarse, gain fine):
//   rho = softmax(s over present branches), d rho_i = g x_i,
//   ds_i = rho_i (d rho_i - sum_j rho_j d rho_j),
//   d local = 2 g rho_0, d coarse = gain g rho_1, d fine = gain g rho_2,
//   d raw_q += sum_i ds_i a_i, d fusion_a_i += ds_i raw_q, d fusion_b_i += ds_i.
// Rows without history (output = local): d local = g.
// Also: dnum = d fine / den, dden = -sum_e d fine fine / den, the local
// attention's delta = sum_e d local * local, and d alpha = 2 sum g (rho_1
// coarse + rho_2 fine) over fused elements (gain = 2 alpha; the reference
// builds gain from a Python float and has no such gradient).
constexpr int kFuseChunk = 64;      // tokens per fuse_bwd_kernel workgroup
constexpr int kFuseVecChunk = 256;  // tokens per fuse_bwd_vec_kernel workgroup

template <int D>
__global__ __launch_bounds__(kThreads) void fuse_bwd_kernel(TrainBwdParams p) {
  constexpr int ROWS = kThreads / D;            // tokens in flight per workgroup
  __shared__ float red[3][kThreads / 64];       // per-wave partials (delta, dden, sum exp)
  __shared__ float facc[6][ROWS][D];            // dfa, dfb partials per lane row
  const int chunks = (p.T + kFuseChunk - 1) / kFuseChunk;
  const int h = blockIdx.x % p.H;
  const int b = (blockIdx.x / p.H) % p.B;
  const int chunk = blockIdx.x / (p.H * p.B);
  (void)chunks;
  const int tid = threadIdx.x, e = tid % D, r = tid / D, lane = tid & 63, w = tid >> 6;
  float a[3], bb[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    a[i] = rbf(load_param(p.fa, p.f_dtype, h * p.fa_s[0] + e * p.fa_s[1] + i * p.fa_s[2]));
    bb[i] = rbf(load_param(p.fb, p.f_dtype, h * p.fb_s[0] + e * p.fb_s[1] + i * p.fb_s[2]));
  }
  float sfa[3] = {0.f, 0.f, 0.f}, sfb[3] = {0.f, 0.f, 0.f};
  float sgain = 0.0f;
  // The next ROWS tokens' inputs are loaded before this step's outputs are
  // stored (the loads cannot pass the stores otherwise: the buffers may alias).
  struct In { float g, L, x, C, F, den; };
  const int t_beg = chunk * kFuseChunk, t_end = min(p.T, (chunk + 1) * kFuseChunk);
  auto load_in = [&](int t0) __attribute__((always_inline)) {
    In v;
    const int t = t0 + r;
    const bool on = t < t_end;
    const int tt = on ? t : t0;
    const size_t row = ((size_t)b * p.T + tt) * p.H + h;
    const bool fine_on = on && t >= p.first_fine;
    const bool coarse_on = fine_on && p.coarse_values && t >= p.first_coarse;
    v.g = on ? bf2f(p.grad[b * p.g_sb + (int64_t)tt * p.g_st + h * p.g_sh + e]) : 0.0f;
    v.L = bf2f(p.local[row * D + e]);
    v.x = bf2f(p.rq.p[b * p.rq.sb + (int64_t)tt * p.rq.st + h * p.rq.sh + e]);
    v.C = coarse_on ? bf2f(p.coarse[row * D + e]) : 0.0f;
    v.F = fine_on ? bf2f(p.fine[row * D + e]) : 0.0f;
    v.den = fine_on ? p.den[row] : 1.0f;
    return v;
  };
  In cur = {0.f, 0.f, 0.f, 0.f, 0.f, 1.f};
  if (t_beg < t_end) cur = load_in(t_beg);
  for (int t0 = t_beg; t0 < t_end; t0 += ROWS) {
    In nxt = cur;
    if (t0 + ROWS < t_end) nxt = load_in(t0 + ROWS);
    const int t = t0 + r;
    const bool on = t < t_end;
    const size_t row = ((size_t)b * p.T + (on ? t : t0)) * p.H + h;
    const float g = cur.g;
    const float L = cur.L;
    const bool fine_on = t >= p.first_fine;
    const bool coarse_on = p.coarse_values && t >= p.first_coarse;
    float dlocal = g, dden_part = 0.0f;
    if (on && fine_on) {
      const float x = cur.x;
      const float C = cur.C;
      const float F = cur.F;
      const float den = cur.den;
      float s[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) s[i] = rbf(rbf(a[i] * x) + bb[i]);
      s[0] = rbf(s[0] + (coarse_on ? kLogTwoBf16 : 0.0f));
      const float top = coarse_on ? fmaxf(s[0], fmaxf(s[1], s[2])) : fmaxf(s[0], s[2]);
      float rho[3];
      rho[0] = __expf(s[0] - top);
      rho[1] = coarse_on ? __expf(s[1] - top) : 0.0f;
      rho[2] = __expf(s[2] - top);
      const float inv = 1.0f / (rho[0] + rho[1] + rho[2]);
#pragma unroll
      for (int i = 0; i < 3; ++i) rho[i] *= inv;
      const float xv[3] = {rbf(2.0f * L), rbf(p.gain * C), rbf(p.gain * F)};
      float dr[3], mean = 0.0f;
#pragma unroll
      for (int i = 0; i < 3; ++i) { dr[i] = g * xv[i]; mean += rho[i] * dr[i]; }
      float drq = 0.0f;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const float ds = rho[i] * (dr[i] - mean);
        drq += ds * a[i];
        sfa[i] += ds * x;
        sfb[i] += ds;
      }
      dlocal = 2.0f * g * rho[0];
      sgain += g * (rho[1] * C + rho[2] * F);
      const float dfine = p.gain * g * rho[2];
      p.dcoarse[row * D + e] = p.gain * g * rho[1];
      p.dnum[row * D + e] = dfine / den;
      p.drq[row * D + e] = drq;
      dden_part = -dfine * F / den;
    } else if (on) {
      p.dcoarse[row * D + e] = 0.0f;
      p.dnum[row * D + e] = 0.0f;
      p.drq[row * D + e] = 0.0f;
    }
    if (on) p.dlocal[row * D + e] = f2bf(dlocal);
    // row reductions over e: D = 64 is one wave, D = 128 two waves
    const float xq = cur.x;
    float mx = wave_max(xq);
    if constexpr (D == 128) {
      if (lane == 0) red[0][w] = mx;
      __syncthreads();
      mx = fmaxf(red[0][w & ~1], red[0][w | 1]);
      __syncthreads();
    }
    const float ex = __expf(xq - mx);
    float dl = wave_sum_fold(on ? dlocal * L : 0.0f);
    float dd = wave_sum_fold(dden_part);
    float sx = wave_sum_fold(ex);
    if constexpr (D == 128) {
      if (lane == 0) { red[0][w] = dl; red[1][w] = dd; red[2][w] = sx; }
      __syncthreads();
      dl = red[0][w & ~1] + red[0][w | 1];
      dd = red[1][w & ~1] + red[1][w | 1];
      sx = red[2][w & ~1] + red[2][w | 1];
      __syncthreads();
    }
    if (on) p.h[row * D + e] = f2bf(ex / sx);
    if (on && e == 0) {
      p.delta[row] = dl;
      p.dden[row] = dd;
    }
    cur = nxt;
  }
  if (p.dalpha_parts) {
    // one partial per workgroup (a single contended atomic serialised ~12K
    // waves); dalpha_kernel adds them in a fixed order
    const float sg = wave_sum_fold(sgain);
    if (lane == 0) red[0][w] = sg;
    __syncthreads();
    if (tid == 0) {
      float t = 0.0f;
      for (int i = 0; i < kThreads / 64; ++i) t += red[0][i];
      p.dalpha_parts[blockIdx.x] = 2.0f * t;
    }
  }
  // d fusion_a / d fusion_b: sum the ROWS lane rows, one atomic per (e, i).
#pragma unroll
  for (int i = 0; i < 3; ++i) { facc[i][r][e] = sfa[i]; facc[3 + i][r][e] = sfb[i]; }
  __syncthreads();
  for (int j = tid; j < 6 * D; j += kThreads) {
    const int k = j / D, ee = j % D;
    float s = 0.0f;
    for (int rr = 0; rr < ROWS; ++rr) s += facc[k][rr][ee];
    float* dst = k < 3 ? p.dfa : p.dfb;
    atomicAdd(dst + (h * D + ee) * 3 + (k % 3), s);
  }
}

// The same adjoint with eight channels per lane: lane row r = one token, its
// D / 8 lanes (contiguous in the wave) hold channels 8 c .. 8 c + 8 as 16-byte
// loads and stores, and the row reductions (softmax of raw_q, delta, dden)
// take log2(D / 8) shuffles. Needs 16-byte aligned rows (every bf16 row
// stride a multiple of 8); launch_fuse_bwd checks and otherwise runs
// fuse_bwd_kernel. A workgroup takes kFuseVecChunk tokens (fewer workgroups
// than fuse_bwd_kernel: the per-workgroup set-up and d fusion sums amortise
// over more rows); one d alpha partial per workgroup as there.
TAO_DEV void load_bf8(const bf16_t* src, float out[8]) {
  const uint4 u = *(const uint4*)src;
  const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(wv[i] << 16);
    out[2 * i + 1] = __uint_as_float(wv[i] & 0xFFFF0000u);
  }
}

TAO_DEV void store_bf8(bf16_t* dst, const float v[8]) {
  uint32_t wv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wv[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
  *(uint4*)dst = make_uint4(wv[0], wv[1], wv[2], wv[3]);
}

TAO_DEV void store_f8(float* dst, const float v[8]) {
  *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
  *(float4*)(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

template <int LPR>
TAO_DEV float row_sum(float v) {
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int LPR>
TAO_DEV float row_max(float v) {
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

template <int D>
__global__ __launch_bounds__(kThreads) void fuse_bwd_vec_kernel(TrainBwdParams p) {
  constexpr int LPR = D / 8, RPW = 64 / LPR, NW = kThreads / 64, ROWS = NW * RPW;
  __shared__ float facc[6][NW][D];               // dfa, dfb per wave
  __shared__ float red[NW];
  const int h = blockIdx.x % p.H;
  const int b = (blockIdx.x / p.H) % p.B;
  const int chunk = blockIdx.x / (p.H * p.B);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int cl = lane % LPR, r = w * RPW + lane / LPR, e0 = 8 * cl;
  float a[3][8], bb[3][8], sfa[3][8], sfb[3][8];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a[i][j] = rbf(load_param(p.fa, p.f_dtype, h * p.fa_s[0] + (e0 + j) * p.fa_s[1] + i * p.fa_s[2]));
      bb[i][j] = rbf(load_param(p.fb, p.f_dtype, h * p.fb_s[0] + (e0 + j) * p.fb_s[1] + i * p.fb_s[2]));
      sfa[i][j] = 0.0f;
      sfb[i][j] = 0.0f;
    }
  float sgain = 0.0f;
  const int t_beg = chunk * kFuseVecChunk, t_end = min(p.T, (chunk + 1) * kFuseVecChunk);
  for (int t0 = t_beg; t0 < t_end; t0 += ROWS) {
    const int t = t0 + r;
    const bool on = t < t_end;
    const int tt = on ? t : t0;
    const size_t row = ((size_t)b * p.T + tt) * p.H + h;
    const bool fine_on = on && t >= p.first_fine;
    const bool coarse_on = fine_on && p.coarse_values && t >= p.first_coarse;
    float g[8], L[8], x[8], C[8], F[8];
    load_bf8(p.grad + b * p.g_sb + (int64_t)tt * p.g_st + h * p.g_sh + e0, g);
    load_bf8(p.local + row * D + e0, L);
    load_bf8(p.rq.p + b * p.rq.sb + (int64_t)tt * p.rq.st + h * p.rq.sh + e0, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) { C[j] = 0.0f; F[j] = 0.0f; if (!on) g[j] = 0.0f; }
    if (coarse_on) load_bf8(p.coarse + row * D + e0, C);
    if (fine_on) load_bf8(p.fine + row * D + e0, F);
    const float den = fine_on ? p.den[row] : 1.0f;
    float dlocal[8], dco[8], dnu[8], drq[8], dden_part = 0.0f, dl_part = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      dlocal[j] = g[j];
      dco[j] = 0.0f;
      dnu[j] = 0.0f;
      drq[j] = 0.0f;
    }
    if (fine_on) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float sc[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) sc[i] = rbf(rbf(a[i][j] * x[j]) + bb[i][j]);
        sc[0] = rbf(sc[0] + (coarse_on ? kLogTwoBf16 : 0.0f));
        const float top = coarse_on ? fmaxf(sc[0], fmaxf(sc[1], sc[2])) : fmaxf(sc[0], sc[2]);
        float rho[3];
        rho[0] = __expf(sc[0] - top);
        rho[1] = coarse_on ? __expf(sc[1] - top) : 0.0f;
        rho[2] = __expf(sc[2] - top);
        const float inv = 1.0f / (rho[0] + rho[1] + rho[2]);
#pragma unroll
        for (int i = 0; i < 3; ++i) rho[i] *= inv;
        const float xv[3] = {rbf(2.0f * L[j]), rbf(p.gain * C[j]), rbf(p.gain * F[j])};
        float dr[3], mean = 0.0f;
#pragma unroll
        for (int i = 0; i < 3; ++i) { dr[i] = g[j] * xv[i]; mean += rho[i] * dr[i]; }
        float dq = 0.0f;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          const float ds = rho[i] * (dr[i] - mean);
          dq += ds * a[i][j];
          sfa[i][j] += ds * x[j];
          sfb[i][j] += ds;
        }
        dlocal[j] = 2.0f * g[j] * rho[0];
        sgain += g[j] * (rho[1] * C[j] + rho[2] * F[j]);
        const float dfine = p.gain * g[j] * rho[2];
        dco[j] = p.gain * g[j] * rho[1];
        dnu[j] = dfine / den;
        drq[j] = dq;
        dden_part -= dfine * F[j] / den;
      }
    }
    if (on) {
      store_f8(p.dcoarse + row * D + e0, dco);
      store_f8(p.dnum + row * D + e0, dnu);
      store_f8(p.drq + row * D + e0, drq);
      store_bf8(p.dlocal + row * D + e0, dlocal);
#pragma unroll
      for (int j = 0; j < 8; ++j) dl_part += dlocal[j] * L[j];
    }
    // h = softmax_D(raw_q) and the row sums (the row's LPR lanes)
    float mx = x[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) mx = fmaxf(mx, x[j]);
    mx = row_max<LPR>(mx);
    float ex[8], sx = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) { ex[j] = __expf(x[j] - mx); sx += ex[j]; }
    sx = row_sum<LPR>(sx);
    const float dl = row_sum<LPR>(dl_part);
    const float dd = row_sum<LPR>(dden_part);
    if (on) {
      float hv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) hv[j] = ex[j] / sx;
      store_bf8(p.h + row * D + e0, hv);
      if (cl == 0) {
        p.delta[row] = dl;
        p.dden[row] = dd;
      }
    }
  }
  if (p.dalpha_parts) {
    const float sg = wave_sum_fold(sgain);
    if (lane == 0) red[w] = sg;
    __syncthreads();
    if (tid == 0) {
      float t = 0.0f;
      for (int i = 0; i < NW; ++i) t += red[i];
      p.dalpha_parts[blockIdx.x] = 2.0f * t;
    }
  }
  // d fusion_a / d fusion_b: the wave's rows (lanes cl, cl + LPR, ...) by
  // shuffles, then the waves in LDS, one atomic per (e, i).
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float va = sfa[i][j], vb = sfb[i][j];
#pragma unroll
      for (int off = LPR; off < 64; off <<= 1) {
        va += __shfl_xor(va, off, 64);
        vb += __shfl_xor(vb, off, 64);
      }
      if (lane < LPR) { facc[i][w][e0 + j] = va; facc[3 + i][w][e0 + j] = vb; }
    }
  __syncthreads();
  for (int j = tid; j < 6 * D; j += kThreads) {
    const int k = j / D, ee = j % D;
    float sum = 0.0f;
    for (int ww = 0; ww < NW; ++ww) sum += facc[k][ww][ee];
    float* dst = k < 3 ? p.dfa : p.dfb;
    atomicAdd(dst + (h * D + ee) * 3 + (k % 3), sum);
  }
}

// d alpha: the workgroups' partials in index order (one workgroup).
__global__ __launch_bounds__(256) void dalpha_kernel(const float* parts, int n, float* out) {
  __shared__ float red[4];
  float s = 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) s += parts[i];
  s = wave_sum_fold(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) *out = (red[0] + red[1]) + (red[2] + red[3]);
}

// ---------------------------------------------------------------------------
// Local attention adjoints (flash_attention.py:16-37 through autograd) with
// the full-sequence windows: query q sees keys [max(0, F tile(q) - keep), q].
// P = 2^(s c - lse2) from the forward's saved log2-sum-exp (c = log2 e /
// sqrt(D)), dS = P (dP - delta), dP = dO V^T; dQ = dS K / sqrt(D),
// dK = dS^T Q / sqrt(D), dV = P^T dO.
// dK / dV: at D64, 256 keys (one tile) per workgroup, so each staged query
// block serves 8 waves of keys; D128 keeps 128 keys (4 waves) within 256
// VGPRs per lane.
template <int D> constexpr int kDkvWaves = D == 64 ? 8 : 4;
template <int D> constexpr int kDkvThreads = 64 * kDkvWaves<D>;
// dQ likewise: 256 queries per workgroup at D64, 128 at D128.
template <int D> constexpr int kDqWaves = D == 64 ? 8 : 4;
template <int D> constexpr int kDqThreads = 64 * kDqWaves<D>;
constexpr int kBwdKeys = 64;          // keys per staged block (dQ pass)
constexpr int kBwdQ = 64;             // queries per staged block (dK/dV pass)

// Window geometry of the HIP path (fine_tokens 256, local_keep 512; the
// launcher rejects others).
constexpr int kFt = 256, kKeep = 512;

TAO_DEV long long window_start(long long q, int, int) {
  const long long s = ((q >> 8) << 8) - kKeep;
  return s > 0 ? s : 0;
}

// dQ pass: workgroup = 128 queries of one (batch, head); wave w owns 32.
template <int D>
struct DqSmem {
  bf16_t k[kBwdKeys][D + 8];
  bf16_t v[kBwdKeys][D + 8];
  bf16_t kt[D][kBwdKeys + 4];
};

template <int D>
__global__ __launch_bounds__(kDqThreads<D>) void attn_bwd_dq_kernel(AttnBwdParams p) {
  __shared__ DqSmem<D> sm;
  constexpr int CH = D / 8, DT = D / 32, KK = D / 16;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int b = bh / p.H, h = bh % p.H;
  const long long first = (long long)(blockIdx.x / BH) * (kDqWaves<D> * 32);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const int count = (int)min((long long)kDqWaves<D> * 32, (long long)p.T - first);
  const int nq = min(max(count - wave * 32, 0), 32);
  const long long qtok = first + (nq > 0 ? wave * 32 + min(li, nq - 1) : 0);
  const long long wave_first = first + wave * 32, wave_last = wave_first + nq - 1;
  const long long kstart = window_start(first, p.ft, p.keep);
  const long long kend = first + count;                 // exclusive
  bf16x8 qreg[KK], oreg[KK];
  {
    const bf16_t* qrow = p.q.p + b * p.q.sb + qtok * p.q.st + h * p.q.sh;
    const bf16_t* orow = p.dout + ((size_t)b * p.T + qtok) * p.H * D + (size_t)h * D;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      qreg[kk] = as_bf16x8(*(const uint4*)(qrow + 16 * kk + 8 * hl));
      oreg[kk] = as_bf16x8(*(const uint4*)(orow + 16 * kk + 8 * hl));
    }
  }
  const size_t qrowi = ((size_t)b * p.T + qtok) * p.H + h;
  const float lse2 = p.lse[qrowi], dlt = p.delta[qrowi];
  const long long ws = window_start(qtok, p.ft, p.keep);
  const int ws_last = (int)window_start(wave_last, p.ft, p.keep);   // latest window start
  const float scale_log2 = (float)(1.4426950408889634 / __builtin_sqrt((double)D));
  floatx16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
  // The next key block's rows wait in registers while this one computes.
  constexpr int KJ = kBwdKeys * CH / kDqThreads<D>;
  static_assert(KJ * kDqThreads<D> == kBwdKeys * CH, "whole jobs per thread");
  uint4 kpre[KJ], vpre[KJ];
  auto fetch = [&](long long kb) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int job = tid + j * kDqThreads<D>, r = job / CH, c = job % CH;
      kpre[j] = make_uint4(0, 0, 0, 0);
      vpre[j] = make_uint4(0, 0, 0, 0);
      if (kb + r < kend) {
        kpre[j] = *(const uint4*)(p.k.p + b * p.k.sb + (kb + r) * p.k.st + h * p.k.sh + c * 8);
        vpre[j] = *(const uint4*)(p.v.p + b * p.v.sb + (kb + r) * p.v.st + h * p.v.sh + c * 8);
      }
    }
  };
  fetch(kstart);
  for (long long kb = kstart; kb < kend; kb += kBwdKeys) {
    __syncthreads();
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int job = tid + j * kDqThreads<D>, r = job / CH, c = job % CH;
      *(uint4*)&sm.k[r][c * 8] = kpre[j];
      *(uint4*)&sm.v[r][c * 8] = vpre[j];
    }
    __syncthreads();
    if (kb + kBwdKeys < kend) fetch(kb + kBwdKeys);      // overlaps the work below
    // K^T: job = (channel chunk c, key pair)
    for (int job = tid; job < (kBwdKeys / 2) * CH; job += kDqThreads<D>) {
      const int t0 = 2 * (job % (kBwdKeys / 2)), c = job / (kBwdKeys / 2);
      const uint4 ua = *(const uint4*)&sm.k[t0][c * 8];
      const uint4 ub = *(const uint4*)&sm.k[t0 + 1][c * 8];
      const uint32_t wa[4] = {ua.x, ua.y, ua.z, ua.w}, wb[4] = {ub.x, ub.y, ub.z, ub.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *(uint32_t*)&sm.kt[c * 8 + 2 * i][t0] = (wa[i] & 0xFFFFu) | (wb[i] << 16);
        *(uint32_t*)&sm.kt[c * 8 + 2 * i + 1][t0] = (wa[i] >> 16) | (wb[i] & 0xFFFF0000u);
      }
    }
    __syncthreads();
    if (nq == 0 || kb > wave_last || kb + kBwdKeys <= window_start(wave_first, p.ft, p.keep))
      continue;
    floatx16 s[2], dp[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
      for (int i = 0; i < 16; ++i) { s[sub][i] = 0.0f; dp[sub][i] = 0.0f; }
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const bf16x8 ak = as_bf16x8(*(const uint4*)&sm.k[sub * 32 + li][16 * kk + 8 * hl]);
        const bf16x8 av = as_bf16x8(*(const uint4*)&sm.v[sub * 32 + li][16 * kk + 8 * hl]);
        s[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ak, qreg[kk], s[sub], 0, 0, 0);
        dp[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, oreg[kk], dp[sub], 0, 0, 0);
      }
    }
    // S^T layout: lane holds query li, keys 8 (i / 4) + 4 hl + i % 4 of each
    // sub-tile. A sub-tile wholly inside every query's window (and before
    // every query) needs no mask; the others test 32-bit positions.
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int k_lo = (int)(kb + sub * 32);
      const bool full = nq == 32 && k_lo + 31 <= (int)wave_first && k_lo >= ws_last &&
                        k_lo + 31 < (int)kend;                         // wave-uniform
      if (full) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float pv = __builtin_amdgcn_exp2f(fmaf(s[sub][i], scale_log2, -lse2));
          s[sub][i] = pv * (dp[sub][i] - dlt);          // dS^T
        }
      } else {
        const int qt = (int)qtok, wsi = (int)ws, ke = (int)kend;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = k_lo + 8 * (i / 4) + 4 * hl + (i % 4);
          const bool ok = li < nq && key <= qt && key >= wsi && key < ke;
          const float pv = ok ? __builtin_amdgcn_exp2f(fmaf(s[sub][i], scale_log2, -lse2)) : 0.0f;
          s[sub][i] = pv * (dp[sub][i] - dlt);
        }
      }
    }
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        uint32_t packed[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          packed[j] = pack_bf16x2(s[sub][8 * half + 2 * j], s[sub][8 * half + 2 * j + 1]);
        const bf16x8 pb = as_bf16x8(make_uint4(packed[0], packed[1], packed[2], packed[3]));
        const int kbase = sub * 32 + 16 * half + 4 * hl;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const uint2 lo = *(const uint2*)&sm.kt[t * 32 + li][kbase];
          const uint2 hi = *(const uint2*)&sm.kt[t * 32 + li][kbase + 8];
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y)), pb, acc[t], 0, 0, 0);
        }
      }
  }
  if (li >= nq) return;
  const float scale = (float)(1.0 / __builtin_sqrt((double)D));
  bf16_t* dq = p.dq + qrowi * D;
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const int d = t * 32 + 8 * (i / 4) + 4 * hl;
      uint2 packed;
      packed.x = pack_bf16x2(acc[t][i] * scale, acc[t][i + 1] * scale);
      packed.y = pack_bf16x2(acc[t][i + 2] * scale, acc[t][i + 3] * scale);
      *(uint2*)(dq + d) = packed;
    }
}

// dK / dV pass: workgroup = 128 keys of one (batch, head); wave w owns 32.
// Queries that see a key k lie in [k, F (tile(k) + 1) + keep).
template <int D>
struct DkvSmem {
  bf16_t q[kBwdQ][D + 8];
  bf16_t o[kBwdQ][D + 8];          // dO rows
  bf16_t qt[D][kBwdQ + 4];
  bf16_t ot[D][kBwdQ + 4];
  float lse[kBwdQ], dl[kBwdQ];
};

template <int D>
__global__ __launch_bounds__(kDkvThreads<D>) void attn_bwd_dkv_kernel(AttnBwdParams p) {
  __shared__ DkvSmem<D> sm;
  constexpr int CH = D / 8, DT = D / 32, KK = D / 16;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int b = bh / p.H, h = bh % p.H;
  const long long first = (long long)(blockIdx.x / BH) * (kDkvWaves<D> * 32);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const int count = (int)min((long long)kDkvWaves<D> * 32, (long long)p.T - first);
  const int nk = min(max(count - wave * 32, 0), 32);
  const long long ktok = first + (nk > 0 ? wave * 32 + min(li, nk - 1) : 0);
  const long long qend = min((long long)p.T, ((first >> 8) + 1) * kFt + kKeep);
  bf16x8 kreg[KK], vreg[KK];
  {
    const bf16_t* krow = p.k.p + b * p.k.sb + ktok * p.k.st + h * p.k.sh;
    const bf16_t* vrow = p.v.p + b * p.v.sb + ktok * p.v.st + h * p.v.sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      kreg[kk] = as_bf16x8(*(const uint4*)(krow + 16 * kk + 8 * hl));
      vreg[kk] = as_bf16x8(*(const uint4*)(vrow + 16 * kk + 8 * hl));
    }
  }
  const float scale_log2 = (float)(1.4426950408889634 / __builtin_sqrt((double)D));
  floatx16 dk[DT], dv[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) { dk[t][i] = 0.0f; dv[t][i] = 0.0f; }
  // The next query block's rows wait in registers while this one computes.
  constexpr int QJ = kBwdQ * CH / kDkvThreads<D>;
  static_assert(QJ * kDkvThreads<D> == kBwdQ * CH, "whole jobs per thread");
  uint4 qpre[QJ], opre[QJ];
  float lpre = 0.0f, dpre = 0.0f;
  auto fetch = [&](long long qb) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < QJ; ++j) {
      const int job = tid + j * kDkvThreads<D>, r = job / CH, c = job % CH;
      qpre[j] = make_uint4(0, 0, 0, 0);
      opre[j] = make_uint4(0, 0, 0, 0);
      if (qb + r < qend) {
        qpre[j] = *(const uint4*)(p.q.p + b * p.q.sb + (qb + r) * p.q.st + h * p.q.sh + c * 8);
        opre[j] = *(const uint4*)(p.dout + (((size_t)b * p.T + qb + r) * p.H + h) * D + c * 8);
      }
    }
    if (tid < kBwdQ) {
      const long long qq = qb + tid;
      const size_t row = ((size_t)b * p.T + (qq < qend ? qq : qb)) * p.H + h;
      lpre = qq < qend ? p.lse[row] : 0.0f;
      dpre = qq < qend ? p.delta[row] : 0.0f;
    }
  };
  fetch(first);
  for (long long qb = first; qb < qend; qb += kBwdQ) {
    __syncthreads();
#pragma unroll
    for (int j = 0; j < QJ; ++j) {
      const int job = tid + j * kDkvThreads<D>, r = job / CH, c = job % CH;
      *(uint4*)&sm.q[r][c * 8] = qpre[j];
      *(uint4*)&sm.o[r][c * 8] = opre[j];
    }
    if (tid < kBwdQ) {
      sm.lse[tid] = lpre;
      sm.dl[tid] = dpre;
    }
    __syncthreads();
    if (qb + kBwdQ < qend) fetch(qb + kBwdQ);            // overlaps the work below
    for (int job = tid; job < (kBwdQ / 2) * CH; job += kDkvThreads<D>) {
      const int t0 = 2 * (job % (kBwdQ / 2)), c = job / (kBwdQ / 2);
      const uint4 qa = *(const uint4*)&sm.q[t0][c * 8], qb2 = *(const uint4*)&sm.q[t0 + 1][c * 8];
      const uint4 oa = *(const uint4*)&sm.o[t0][c * 8], ob = *(const uint4*)&sm.o[t0 + 1][c * 8];
      const uint32_t wqa[4] = {qa.x, qa.y, qa.z, qa.w}, wqb[4] = {qb2.x, qb2.y, qb2.z, qb2.w};
      const uint32_t woa[4] = {oa.x, oa.y, oa.z, oa.w}, wob[4] = {ob.x, ob.y, ob.z, ob.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *(uint32_t*)&sm.qt[c * 8 + 2 * i][t0] = (wqa[i] & 0xFFFFu) | (wqb[i] << 16);
        *(uint32_t*)&sm.qt[c * 8 + 2 * i + 1][t0] = (wqa[i] >> 16) | (wqb[i] & 0xFFFF0000u);
        *(uint32_t*)&sm.ot[c * 8 + 2 * i][t0] = (woa[i] & 0xFFFFu) | (wob[i] << 16);
        *(uint32_t*)&sm.ot[c * 8 + 2 * i + 1][t0] = (woa[i] >> 16) | (wob[i] & 0xFFFF0000u);
      }
    }
    __syncthreads();
    // keys of this wave: [kw, kw + nk); queries of the block: [qb, qb + 64)
    const long long kw = first + wave * 32;
    if (nk == 0 || qb + kBwdQ <= kw) continue;          // all queries before the keys
    // One 32-query sub-block at a time (keeps S, dP and P of one block live).
#pragma unroll 1
    for (int sub = 0; sub < 2; ++sub) {
      if (qb + sub * 32 >= qend || qb + sub * 32 + 31 < kw) continue;   // uniform
      floatx16 sv, dpv;
#pragma unroll
      for (int i = 0; i < 16; ++i) { sv[i] = 0.0f; dpv[i] = 0.0f; }
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const bf16x8 aq = as_bf16x8(*(const uint4*)&sm.q[sub * 32 + li][16 * kk + 8 * hl]);
        const bf16x8 ao = as_bf16x8(*(const uint4*)&sm.o[sub * 32 + li][16 * kk + 8 * hl]);
        sv = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, kreg[kk], sv, 0, 0, 0);
        dpv = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ao, vreg[kk], dpv, 0, 0, 0);
      }
      // S layout: lane holds key li, queries 8 (i / 4) + 4 hl + i % 4 of the
      // sub-block. A sub-block whose every query sees every key of the wave
      // needs no mask; the others test 32-bit positions.
      float pm[16];
      const int q_lo = (int)(qb + sub * 32);
      const bool full = nk == 32 && (int)kw + 31 <= q_lo && q_lo + 31 < (int)qend &&
                        (int)kw >= (int)window_start(q_lo + 31, p.ft, p.keep);   // wave-uniform
      if (full) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int qo = sub * 32 + 8 * (i / 4) + 4 * hl + (i % 4);
          const float pv = __builtin_amdgcn_exp2f(fmaf(sv[i], scale_log2, -sm.lse[qo]));
          pm[i] = pv;
          sv[i] = pv * (dpv[i] - sm.dl[qo]);          // dS
        }
      } else {
        const int kt = (int)ktok, qe = (int)qend;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int qo = sub * 32 + 8 * (i / 4) + 4 * hl + (i % 4);
          const int qq = q_lo + 8 * (i / 4) + 4 * hl + (i % 4);
          const int wsq = ((qq >> 8) << 8) - kKeep;
          const bool ok = li < nk && qq < qe && kt <= qq && kt >= wsq;
          const float pv = ok ? __builtin_amdgcn_exp2f(fmaf(sv[i], scale_log2, -sm.lse[qo])) : 0.0f;
          pm[i] = pv;
          sv[i] = pv * (dpv[i] - sm.dl[qo]);
        }
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        uint32_t pp[4], dd[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pp[j] = pack_bf16x2(pm[8 * half + 2 * j], pm[8 * half + 2 * j + 1]);
          dd[j] = pack_bf16x2(sv[8 * half + 2 * j], sv[8 * half + 2 * j + 1]);
        }
        const bf16x8 pb = as_bf16x8(make_uint4(pp[0], pp[1], pp[2], pp[3]));
        const bf16x8 db = as_bf16x8(make_uint4(dd[0], dd[1], dd[2], dd[3]));
        const int kbase = sub * 32 + 16 * half + 4 * hl;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const uint2 olo = *(const uint2*)&sm.ot[t * 32 + li][kbase];
          const uint2 ohi = *(const uint2*)&sm.ot[t * 32 + li][kbase + 8];
          dv[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              as_bf16x8(make_uint4(olo.x, olo.y, ohi.x, ohi.y)), pb, dv[t], 0, 0, 0);
          const uint2 qlo = *(const uint2*)&sm.qt[t * 32 + li][kbase];
          const uint2 qhi = *(const uint2*)&sm.qt[t * 32 + li][kbase + 8];
          dk[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              as_bf16x8(make_uint4(qlo.x, qlo.y, qhi.x, qhi.y)), db, dk[t], 0, 0, 0);
        }
      }
    }
  }
  if (li >= nk) return;
  const float scale = (float)(1.0 / __builtin_sqrt((double)D));
  const size_t krowi = ((size_t)b * p.T + ktok) * p.H + h;
  bf16_t* dkp = p.dk + krowi * D;
  float* dvp = p.dv + krowi * D;
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const int d = t * 32 + 8 * (i / 4) + 4 * hl;
      uint2 packed;
      packed.x = pack_bf16x2(dk[t][i] * scale, dk[t][i + 1] * scale);
      packed.y = pack_bf16x2(dk[t][i + 2] * scale, dk[t][i + 3] * scale);
      *(uint2*)(dkp + d) = packed;
      *(float4*)(dvp + d) = make_float4(dv[t][i], dv[t][i + 1], dv[t][i + 2], dv[t][i + 3]);
    }
}

// ---------------------------------------------------------------------------
// Memory-branch adjoints (selected_read.py:175-187 and autograd through
// tao_stream.py:530-665). For query q of tile t (V = t - lag visible fines,
// K = V / 8 completed pages, P = K + (V % 8 > 0)), selected fine f on page
// g = f / 8, channel d:
//   a[q][f][d] = h[q][d] pw_t[g][d] sw_t[f][d],
//   num[q] = sum_f a[q][f] C_f,  den[q] = sum_f sum_d a[q][f][d];
// given dnum, dden (fuse_bwd):
//   da = dnum C_f^T + dden,  dC_f += a (x) dnum,
//   dh += da sw pw,  d pw_t[g] += da sw h,  d sw_t[f] += da h pw.
// Tiles of 256 queries share V; lanes are channels (d = lane + 64 k).
constexpr int kRbQ = 128;              // queries per read_bwd workgroup (4 waves x 32)
constexpr int kRbWaves = 4;

TAO_DEV int tile_visible(int t, int lag) { return t > lag ? t - lag : 0; }

template <int D>
struct ReadBwdSmem {
  bf16_t c[2][D][D + 8];               // C (or G) of the current / next fine: [d][e], padded
  float dpw[64][D];                    // d pw of the tile's pages (P <= 64)
  uint32_t bits[512];
  int pre[512];
  int uni[1024];
  uint32_t qw[kRbQ][16];               // the block's selection words (V <= 504)
  int n_union;
};

// Stage X^T (global rows [e][d], d contiguous) as X[d][e] into sm.c.
template <int D>
TAO_DEV void stage_transposed(bf16_t (*c)[D + 8], const bf16_t* src, int tid, int nthreads) {
  constexpr int CH = D / 8;
  for (int job = tid; job < (D / 2) * CH; job += nthreads) {
    const int e0 = 2 * (job % (D / 2)), ch = job / (D / 2);
    const uint4 ua = *(const uint4*)(src + (size_t)e0 * D + ch * 8);
    const uint4 ub = *(const uint4*)(src + (size_t)(e0 + 1) * D + ch * 8);
    const uint32_t wa[4] = {ua.x, ua.y, ua.z, ua.w}, wb[4] = {ub.x, ub.y, ub.z, ub.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *(uint32_t*)&c[ch * 8 + 2 * i][e0] = (wa[i] & 0xFFFFu) | (wb[i] << 16);
      *(uint32_t*)&c[ch * 8 + 2 * i + 1][e0] = (wa[i] >> 16) | (wb[i] & 0xFFFF0000u);
    }
  }
}

// One 256-thread workgroup per (128 queries, batch, head); wave w owns 32
// queries. Per union fine: dA^T... computed as D[q][d] = sum_e dnum[q][e] C[d][e]
// with v_mfma_f32_32x32x16_bf16 (A = the wave's dnum rows in registers, B =
// C rows staged in LDS); the accumulator layout (lane = channel d, 16 query
// rows) carries dden, the selection mask, h, and the dh accumulators.
template <int D>
__global__ __launch_bounds__(kRbWaves * 64) void read_bwd_kernel(MemBwdParams p) {
  constexpr int KK = D / 16, DT = D / 32;
  __shared__ ReadBwdSmem<D> sm;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int b = bh / p.H, h = bh % p.H;
  // Query blocks in reverse order: the latest blocks read the most fines.
  const int q0 = ((int)gridDim.x / BH - 1 - (int)blockIdx.x / BH) * kRbQ;
  const int tile = q0 / p.ft;
  const int V = tile_visible(tile, p.keep / p.ft);
  if (V == 0) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const int G = p.group, K = V / G, P = K + (V % G > 0), erel = V - 1;
  const int nq = min(kRbQ, p.T - q0);
  const int nqw = min(32, max(0, nq - 32 * w));
  const int words = (V + 31) >> 5;
  const bf16_t* pw = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
  const bf16_t* psw = p.psw_pool + ((size_t)erel * BH + bh) * 8 * D;
  const bf16_t* gsw = p.fine_sw + (size_t)bh * p.fine_cap * D;
  // ---- union of the block's selections
  for (int i = tid; i < 512; i += kRbWaves * 64) sm.bits[i] = 0u;
  for (int i = tid; i < 64 * D; i += kRbWaves * 64) (&sm.dpw[0][0])[i] = 0.0f;
  __syncthreads();
  for (int i = tid; i < nq * words; i += kRbWaves * 64) {
    const int qi = i / words, wd = i % words;
    const uint32_t v = p.qsel[((size_t)(b * p.T + q0 + qi) * p.H + h) * p.qsel_words + wd];
    sm.qw[qi][wd] = v;
    if (v) atomicOr(&sm.bits[wd], v);
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int i = 0; i < words; ++i) { sm.pre[i] = run; run += __popc(sm.bits[i]); }
    sm.n_union = run;
  }
  __syncthreads();
  for (int i = tid; i < words; i += kRbWaves * 64) {
    uint32_t bits = sm.bits[i];
    int r = sm.pre[i];
    while (bits) {
      sm.uni[r++] = i * 32 + __ffs(bits) - 1;
      bits &= bits - 1;
    }
  }
  __syncthreads();
  const int U = sm.n_union;
  // ---- the wave's rows: dnum as the MFMA A operand (row li), dden / h in the
  // accumulator layout (rows q_i = 8 (i / 4) + 4 hl + i % 4, column d = 32 t + li)
  const int qa = q0 + 32 * w + (nqw > 0 ? min(li, nqw - 1) : 0);
  const size_t rowa = ((size_t)b * p.T + qa) * p.H + h;
  bf16x8 dn[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    const float* src = p.dnum + rowa * D + 16 * kk + 8 * hl;
    uint32_t pk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) pk[j] = pack_bf16x2(src[2 * j], src[2 * j + 1]);
    dn[kk] = as_bf16x8(make_uint4(pk[0], pk[1], pk[2], pk[3]));
  }
  float dd[16], hd[DT][16], dh[DT][16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int qi = 8 * (i / 4) + 4 * hl + (i % 4);
    const bool ok = qi < nqw;
    const size_t row = ((size_t)b * p.T + q0 + 32 * w + (ok ? qi : 0)) * p.H + h;
    dd[i] = ok ? p.dden[row] : 0.0f;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      hd[t][i] = ok ? bf2f(p.h[row * D + 32 * t + li]) : 0.0f;
      dh[t][i] = 0.0f;
    }
  }
  // The next union fine's C rows are loaded into registers while the current
  // fine is consumed (thread tid owns jobs tid + 256 j of the transposed stage).
  constexpr int JP = (D / 2) * (D / 8) / (kRbWaves * 64);
  static_assert(JP * kRbWaves * 64 == (D / 2) * (D / 8), "stage jobs split evenly");
  uint4 ra[JP], rb[JP];
  auto load_c = [&](int fn) {
    const bf16_t* src = p.bank + ((size_t)bh * p.fine_cap + fn) * D * D;
#pragma unroll
    for (int j = 0; j < JP; ++j) {
      const int job = tid + j * kRbWaves * 64;
      const int e0 = 2 * (job % (D / 2)), ch = job / (D / 2);
      ra[j] = *(const uint4*)(src + (size_t)e0 * D + ch * 8);
      rb[j] = *(const uint4*)(src + (size_t)(e0 + 1) * D + ch * 8);
    }
  };
  if (U > 0) load_c(sm.uni[0]);
  for (int u = 0; u < U; ++u) {
    const int f = sm.uni[u];
    const int g = f / G;
    // Fines alternate between the two C buffers: the barrier below also
    // proves that every wave is done with the fine before the previous one.
    bf16_t (*cu)[D + 8] = sm.c[u & 1];
#pragma unroll
    for (int j = 0; j < JP; ++j) {
      const int job = tid + j * kRbWaves * 64;
      const int e0 = 2 * (job % (D / 2)), ch = job / (D / 2);
      const uint32_t wa[4] = {ra[j].x, ra[j].y, ra[j].z, ra[j].w};
      const uint32_t wb[4] = {rb[j].x, rb[j].y, rb[j].z, rb[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *(uint32_t*)&cu[ch * 8 + 2 * i][e0] = (wa[i] & 0xFFFFu) | (wb[i] << 16);
        *(uint32_t*)&cu[ch * 8 + 2 * i + 1][e0] = (wa[i] >> 16) | (wb[i] & 0xFFFF0000u);
      }
    }
    __syncthreads();
    // selection mask of the wave's 32 queries (bit q)
    const bool mine = li < nqw && ((sm.qw[32 * w + li][f >> 5] >> (f & 31)) & 1u);
    const uint32_t m32 = (uint32_t)(__ballot(mine) & 0xFFFFFFFFull);
    float swv[DT], pwv[DT];
    if (m32 != 0) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const int d = 32 * t + li;
        swv[t] = bf2f(f < K * G ? gsw[(size_t)f * D + d] : psw[(size_t)(f - K * G) * D + d]);
        pwv[t] = bf2f(pw[(size_t)g * D + d]);
      }
    }
    if (u + 1 < U) load_c(sm.uni[u + 1]);
    if (m32 != 0) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        floatx16 da;
#pragma unroll
        for (int i = 0; i < 16; ++i) da[i] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          da = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              dn[kk], as_bf16x8(*(const uint4*)&cu[32 * t + li][16 * kk + 8 * hl]), da, 0, 0, 0);
        float spw = 0.0f, ssw = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int qi = 8 * (i / 4) + 4 * hl + (i % 4);
          const float a = ((m32 >> qi) & 1u) ? da[i] + dd[i] : 0.0f;
          const float dhv = a * swv[t];
          dh[t][i] = fmaf(dhv, pwv[t], dh[t][i]);
          spw = fmaf(dhv, hd[t][i], spw);
          ssw = fmaf(a * hd[t][i], pwv[t], ssw);
        }
        spw += __shfl_xor(spw, 32, 64);
        ssw += __shfl_xor(ssw, 32, 64);
        if (hl == 0) {
          atomicAdd(p.dsw_tile + (((size_t)tile * BH + bh) * p.v_max + f) * D + 32 * t + li, ssw);
          atomicAdd(&sm.dpw[g][32 * t + li], spw);
        }
      }
    }
  }
  // ---- coarse read: dh[q][d] += sum_e dcoarse[q][e] G[d][e] (coarse_pool holds G^T)
  if (p.coarse_values && K >= 1) {
    __syncthreads();
    stage_transposed<D>(sm.c[0], p.coarse_pool + ((size_t)(K - p.coarse_first) * BH + bh) * D * D,
                        tid, kRbWaves * 64);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const float* src = p.dcoarse + rowa * D + 16 * kk + 8 * hl;
      uint32_t pk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) pk[j] = pack_bf16x2(src[2 * j], src[2 * j + 1]);
      dn[kk] = as_bf16x8(make_uint4(pk[0], pk[1], pk[2], pk[3]));
    }
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      floatx16 acc;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            dn[kk], as_bf16x8(*(const uint4*)&sm.c[0][32 * t + li][16 * kk + 8 * hl]), acc, 0, 0,
            0);
#pragma unroll
      for (int i = 0; i < 16; ++i) dh[t][i] += acc[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int qi = 8 * (i / 4) + 4 * hl + (i % 4);
    if (qi < nqw) {
      const size_t row = ((size_t)b * p.T + q0 + 32 * w + qi) * p.H + h;
#pragma unroll
      for (int t = 0; t < DT; ++t) p.dh[row * D + 32 * t + li] = dh[t][i];
    }
  }
  __syncthreads();
  for (int i = tid; i < P * D; i += kRbWaves * 64)
    atomicAdd(p.dpw + (((size_t)tile * BH + bh) * p.pool_pcap + i / D) * D + i % D,
              sm.dpw[i / D][i % D]);
}

TAO_DEV void unpack8f_bwd(const uint4& u, float out[8]) {
  const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(wv[i] << 16);
    out[2 * i + 1] = __uint_as_float(wv[i] & 0xFFFF0000u);
  }
}

// Outer products over a query set: out^T[e][d] = sum_q x[q][e] y[q][d].
// mode 0 (dC of the NF fines f0 .. f0 + NF - 1, f0 = NF * item): queries of
//   every tile that sees f0, x = dnum, y_f = a = h pw sw (zero unless the
//   query selected f); plus the coarse path's share
//   w_f[d] sum_{K > g} cw_K[g][d] dG_K[d][e] for completed f.
// mode 1 (dG of completed count K = coarse_first + item, NF = 1): queries of
//   the tiles with K completed pages, x = dcoarse, y = h.
// Chunks of 32 queries are staged transposed (x^T [e][q] once, y_f^T [d][q]
// per fine: a query's dnum and h rows are read once for all NF fines) and
// reduced with v_mfma_f32_32x32x16_bf16 (m = e, n = d, k = q); wave w owns
// output tiles w, w + 4, ... of the (D / 32)^2 tiles of every fine. A
// workgroup takes kObTiles (dC) or kObTilesG (dG) of an item's tiles (grid =
// items x tile groups x B*H) and adds its sums into the zeroed output with
// fp32 atomics; the first group adds the coarse share.
constexpr int kObQ = 32;
constexpr int kObTiles = 2;    // query tiles per dC workgroup (mode 0)
constexpr int kObTilesG = 1;   // query tiles per dG workgroup (mode 1: few items, more groups)
template <int D> constexpr int kObFines = D == 64 ? 4 : 2;

template <int D, int NF>
__global__ __launch_bounds__(kThreads) void outer_bwd_kernel(MemBwdParams p, int mode) {
  constexpr int DT = D / 32, NT = DT * DT, TPW = (NT + 3) / 4;
  static_assert(32 % NF == 0, "a fine group's selection bits share one word");
  // Chunks alternate between two staging buffers, so one barrier per chunk
  // separates its staging from its reduction.
  __shared__ bf16_t xt[2][D][kObQ + 8], yt[2][NF][D][kObQ + 8];
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int b = bh / p.H, h = bh % p.H;
  const int G = p.group, lag = p.keep / p.ft;
  const int n_tiles = (p.T + p.ft - 1) / p.ft;
  const int tpg = mode == 0 ? kObTiles : kObTilesG;
  const int groups = mode == 0 ? (max(n_tiles - lag - 1, 1) + tpg - 1) / tpg : (G + tpg - 1) / tpg;
  const int item = blockIdx.x / BH / groups, tg = (blockIdx.x / BH) % groups;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  floatx16 acc[NF][TPW];
#pragma unroll
  for (int k = 0; k < NF; ++k)
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[k][j][i] = 0.0f;
  const int f0 = item * NF, Kc = p.coarse_first + item;
  const int t_first = mode == 0 ? f0 + lag + 1 : lag + G * Kc;
  const int t_last = mode == 0 ? n_tiles : min(n_tiles, lag + G * Kc + G);
  const int t_lo = t_first + tg * tpg;
  const int t_hi = min(t_last, t_lo + tpg);
  if (t_lo >= t_hi) return;                          // workgroup-uniform
  const bf16_t* gsw = p.fine_sw + (size_t)bh * p.fine_cap * D;
  // Per tile, the NF fines' page and segment weights (query-independent) in
  // LDS; per 32-query chunk, the next chunk's dnum / h rows and selection
  // bits wait in registers while this chunk is staged and reduced.
  constexpr int JOBS = kObQ * (D / 8) / kThreads;
  static_assert(JOBS * kThreads == kObQ * (D / 8), "whole jobs per thread");
  __shared__ float wpw[NF][D], wsw[NF][D];
  float xpre[JOBS][8];
  uint4 hpre[JOBS];
  uint32_t bpre[JOBS];
  auto fetch = [&](int t, int qb) __attribute__((always_inline)) {
    const int V = tile_visible(t, lag);
    const uint32_t seen = mode == 0 ? ((1u << min(NF, max(V - f0, 0))) - 1u) : 1u;
    const int qb_end = min(p.T, t * p.ft + p.ft);
#pragma unroll
    for (int jb = 0; jb < JOBS; ++jb) {
      const int job = tid + jb * kThreads, qi = job % kObQ, c = job / kObQ;
      const int q = qb + qi;
      uint32_t bits = 0;
      float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
      uint4 hv = make_uint4(0, 0, 0, 0);
      if (q < qb_end) {
        const size_t row = ((size_t)b * p.T + q) * p.H + h;
        bits = mode == 0 ? (p.qsel[row * p.qsel_words + (f0 >> 5)] >> (f0 & 31)) & seen : 1u;
        if (bits) {
          const float* xs = (mode == 0 ? p.dnum : p.dcoarse) + row * D + 8 * c;
          x0 = *(const float4*)xs;
          x1 = *(const float4*)(xs + 4);
          hv = *(const uint4*)(p.h + row * D + 8 * c);
        }
      }
      xpre[jb][0] = x0.x; xpre[jb][1] = x0.y; xpre[jb][2] = x0.z; xpre[jb][3] = x0.w;
      xpre[jb][4] = x1.x; xpre[jb][5] = x1.y; xpre[jb][6] = x1.z; xpre[jb][7] = x1.w;
      hpre[jb] = hv;
      bpre[jb] = bits;
    }
  };
  int t = t_lo, qb = t_lo * p.ft, buf = 0;
  fetch(t, qb);
  while (t < t_hi) {
    const int qa = t * p.ft, qb_end = min(p.T, qa + p.ft);
    if (mode == 0 && qb == qa) {                       // first chunk of tile t
      // every thread is past the previous chunk's staging (the barrier after
      // it), the only reader of wpw / wsw
      const int V = tile_visible(t, lag), erel = V - 1, K = V / G;
      const bf16_t* pw = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
      const bf16_t* psw = p.psw_pool + ((size_t)erel * BH + bh) * 8 * D;
      for (int i = tid; i < NF * D; i += kThreads) {
        const int k = i / D, d = i % D, f = f0 + k;
        const bool vis = f < V;
        wpw[k][d] = vis ? bf2f(pw[(size_t)(f / G) * D + d]) : 0.0f;
        wsw[k][d] = vis ? bf2f(f < K * G ? gsw[(size_t)f * D + d]
                                         : psw[(size_t)(f - K * G) * D + d])
                        : 0.0f;
      }
      __syncthreads();
    }
    // thread = (query qi, 8-channel chunk c): x and y rows, written transposed.
    // A wave's jobs cover all kObQ queries (kObQ divides 64), so its ballot of
    // a fine's selection bits says whether any query of the chunk selects it.
    static_assert(64 % kObQ == 0, "every wave sees every query of the chunk");
    uint32_t any_sel = 0;
#pragma unroll
    for (int k = 0; k < NF; ++k)
      if (__ballot((bpre[0] >> k) & 1u) != 0ull) any_sel |= 1u << k;
#pragma unroll
    for (int jb = 0; jb < JOBS; ++jb) {
      const int job = tid + jb * kThreads, qi = job % kObQ, c = job / kObQ;
      const uint32_t bits = bpre[jb];
      float hv[8];
      unpack8f_bwd(hpre[jb], hv);
#pragma unroll
      for (int j = 0; j < 8; ++j) xt[buf][8 * c + j][qi] = f2bf(xpre[jb][j]);
#pragma unroll
      for (int k = 0; k < NF; ++k) {
        const bool on = (bits >> k) & 1u;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float y = hv[j];
          if (mode == 0) {
            const int d = 8 * c + j;
            y = on ? y * wpw[k][d] * wsw[k][d] : 0.0f;
          }
          yt[buf][k][8 * c + j][qi] = f2bf(y);
        }
      }
    }
    __syncthreads();
    // advance; the next chunk's loads overlap this chunk's MFMAs
    int t2 = t, qb2 = qb + kObQ;
    if (qb2 >= qb_end) { t2 = t + 1; qb2 = t2 * p.ft; }
    if (t2 < t_hi) fetch(t2, qb2);
#pragma unroll
    for (int k = 0; k < NF; ++k) {
      if (!((any_sel >> k) & 1u)) continue;          // workgroup-uniform
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const int tt = w + 4 * j;
        if (tt < NT) {
          const int mt = tt / DT, nt = tt % DT;
#pragma unroll
          for (int ks = 0; ks < kObQ / 16; ++ks)
            acc[k][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                as_bf16x8(*(const uint4*)&xt[buf][32 * mt + li][16 * ks + 8 * hl]),
                as_bf16x8(*(const uint4*)&yt[buf][k][32 * nt + li][16 * ks + 8 * hl]),
                acc[k][j], 0, 0, 0);
        }
      }
    }
    t = t2;
    qb = qb2;
    buf ^= 1;
  }
  const bf16_t* pz = p.page_z + (size_t)bh * p.page_cap * D;
#pragma unroll
  for (int k = 0; k < NF; ++k) {
    const int f = f0 + k;
    if (mode == 0 && f >= p.v_max) break;
    float* out = mode == 0 ? p.dc + ((size_t)bh * p.v_max + f) * D * D
                           : p.dgc + ((size_t)item * BH + bh) * D * D;
    // (Only the softmax writer's page matrices are sums of its fines' C.)
    const bool coarse_share = mode == 0 && tg == 0 && p.coarse_values && !p.values_external &&
                              f < G * (p.v_max / G);
    const int g = f / G;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int tt = w + 4 * j;
      if (tt >= NT) continue;
      const int mt = tt / DT, nt = tt % DT;
      const int d = 32 * nt + li;
      if (coarse_share) {
        const float wf = bf2f(gsw[(size_t)f * D + d]);
        for (int k2 = max(g + 1, p.coarse_first); k2 < p.coarse_first + p.coarse_count; ++k2) {
          float m = -__builtin_inff();
          for (int jj = 0; jj < k2; ++jj) m = fmaxf(m, bf2f(pz[(size_t)jj * D + d]));
          float z = 0.0f;
          for (int jj = 0; jj < k2; ++jj) z += __expf(bf2f(pz[(size_t)jj * D + d]) - m);
          const float scale = wf * __expf(bf2f(pz[(size_t)g * D + d]) - m) / z;
          const float* dg = p.dgc + ((size_t)(k2 - p.coarse_first) * BH + bh) * D * D;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int e = 32 * mt + 8 * (i / 4) + 4 * hl + (i % 4);
            acc[k][j][i] = fmaf(scale, dg[(size_t)e * D + d], acc[k][j][i]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int e = 32 * mt + 8 * (i / 4) + 4 * hl + (i % 4);
        atomicAdd(out + (size_t)e * D + d, acc[k][j][i]);
      }
    }
  }
}

// Page-level adjoints of one tile (softmax over its P pages, the pending
// page's logsumexp and segment weights). Thread per channel.
template <int D>
__global__ __launch_bounds__(D) void page_bwd_kernel(MemBwdParams p) {
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int tile = blockIdx.x / BH;
  const int lag = p.keep / p.ft, G = p.group;
  const int V = tile_visible(tile, lag);
  if (V == 0) return;
  const int d = threadIdx.x;
  const int K = V / G, pend = V % G, P = K + (pend > 0), erel = V - 1;
  const bf16_t* pw = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
  const bf16_t* psw = p.psw_pool + ((size_t)erel * BH + bh) * 8 * D;
  const float* dpw = p.dpw + ((size_t)tile * BH + bh) * p.pool_pcap * D;
  const float* dsw = p.dsw_tile + ((size_t)tile * BH + bh) * p.v_max * D;
  float s = 0.0f;
  for (int g = 0; g < P; ++g) s += bf2f(pw[(size_t)g * D + d]) * dpw[(size_t)g * D + d];
  for (int g = 0; g < K; ++g) {
    const float dpz = bf2f(pw[(size_t)g * D + d]) * (dpw[(size_t)g * D + d] - s);
    atomicAdd(p.dpz + ((size_t)bh * p.page_cap + g) * D + d, dpz);
  }
  for (int f = 0; f < K * G; ++f)
    atomicAdd(p.dsw + ((size_t)bh * p.v_max + f) * D + d, dsw[(size_t)f * D + d]);
  if (pend) {
    float dpend = bf2f(pw[(size_t)K * D + d]) * (dpw[(size_t)K * D + d] - s);
    for (int i = 0; i < pend; ++i)
      dpend -= dsw[(size_t)(K * G + i) * D + d] * bf2f(psw[(size_t)i * D + d]);
    for (int i = 0; i < pend; ++i) {
      const float w = bf2f(psw[(size_t)i * D + d]);
      atomicAdd(p.dz + ((size_t)bh * p.v_max + K * G + i) * D + d,
                dsw[(size_t)(K * G + i) * D + d] * w + dpend * w);
    }
  }
}

// Coarse path, page level, for completed count K (one workgroup per (K, bh),
// thread per channel): cw = softmax over pages < K of page_z,
// d cw[g][d] = sum_e dG[d][e] pc_g[d][e] -> d page_z (softmax adjoint), and
// d w_f[d] = cw[g][d] sum_e dG[d][e] C_f[d][e] -> d sw of f (w_f = sw_f).
// 256 threads: channel d = tid % D, part = tid / D; pages and fines are
// dealt to the parts (the dot products over e are the work), the page dots
// meet in LDS for the softmax adjoint.
constexpr int kCpMaxPages = 64;

template <int D>
__global__ __launch_bounds__(kThreads) void coarse_page_bwd_kernel(MemBwdParams p) {
  constexpr int PARTS = kThreads / D;
  __shared__ float sdcw[kCpMaxPages][D];
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int K = p.coarse_first + blockIdx.x / BH;
  const int d = threadIdx.x % D, part = threadIdx.x / D, G = p.group;
  const bf16_t* pz = p.page_z + (size_t)bh * p.page_cap * D;
  const float* dg = p.dgc + ((size_t)(K - p.coarse_first) * BH + bh) * D * D;   // [e][d]
  auto dot = [&](const bf16_t* mat) __attribute__((always_inline)) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    for (int e = 0; e < D; e += 4) {
      a0 = fmaf(dg[(size_t)e * D + d], bf2f(mat[(size_t)e * D + d]), a0);
      a1 = fmaf(dg[(size_t)(e + 1) * D + d], bf2f(mat[(size_t)(e + 1) * D + d]), a1);
      a2 = fmaf(dg[(size_t)(e + 2) * D + d], bf2f(mat[(size_t)(e + 2) * D + d]), a2);
      a3 = fmaf(dg[(size_t)(e + 3) * D + d], bf2f(mat[(size_t)(e + 3) * D + d]), a3);
    }
    return (a0 + a1) + (a2 + a3);
  };
  for (int g = part; g < K; g += PARTS)
    sdcw[g][d] = dot(p.page_c + ((size_t)bh * p.page_cap + g) * D * D);     // [e][d]
  float m = -__builtin_inff();
  for (int g = 0; g < K; ++g) m = fmaxf(m, bf2f(pz[(size_t)g * D + d]));
  float z = 0.0f;
  for (int g = 0; g < K; ++g) z += __expf(bf2f(pz[(size_t)g * D + d]) - m);
  __syncthreads();
  float s = 0.0f;
  for (int g = 0; g < K; ++g) s += __expf(bf2f(pz[(size_t)g * D + d]) - m) / z * sdcw[g][d];
  for (int g = part; g < K; g += PARTS) {
    const float cw = __expf(bf2f(pz[(size_t)g * D + d]) - m) / z;
    atomicAdd(p.dpz + ((size_t)bh * p.page_cap + g) * D + d, cw * (sdcw[g][d] - s));
  }
  if (p.values_external) {
    // Page matrices not built from the fines' C (regularized writer): their
    // adjoint d page_c[g] += cw[g] * dG (C^T layout), taken by the caller.
    for (int g = part; g < K; g += PARTS) {
      const float cw = __expf(bf2f(pz[(size_t)g * D + d]) - m) / z;
      float* dst = p.dpc + ((size_t)bh * p.dpc_cap + g) * D * D;
      for (int e = 0; e < D; ++e) atomicAdd(dst + (size_t)e * D + d, cw * dg[(size_t)e * D + d]);
    }
    return;
  }
  for (int f = part; f < K * G; f += PARTS) {
    const int g = f / G;
    const float cw = __expf(bf2f(pz[(size_t)g * D + d]) - m) / z;
    const float dw = dot(p.bank + ((size_t)bh * p.fine_cap + f) * D * D);   // C^T [e][d]
    atomicAdd(p.dsw + ((size_t)bh * p.v_max + f) * D + d, cw * dw);
  }
}

// Completed page g: d z of its fines from d sw (global) and d page_z
// (logsumexp adjoint; its softmax weights are the final sw).
template <int D>
__global__ __launch_bounds__(D) void zpage_bwd_kernel(MemBwdParams p) {
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int g = blockIdx.x / BH;
  const int d = threadIdx.x, G = p.group;
  const bf16_t* gsw = p.fine_sw + (size_t)bh * p.fine_cap * D;
  float t1[8], dpz = p.dpz[((size_t)bh * p.page_cap + g) * D + d];
  for (int i = 0; i < G; ++i) {
    const int f = g * G + i;
    t1[i] = p.dsw[((size_t)bh * p.v_max + f) * D + d] * bf2f(gsw[(size_t)f * D + d]);
    dpz -= t1[i];
  }
  for (int i = 0; i < G; ++i) {
    const int f = g * G + i;
    p.dz[((size_t)bh * p.v_max + f) * D + d] += t1[i] + dpz * bf2f(gsw[(size_t)f * D + d]);
  }
}

// Softmax writer adjoint of block f (tao_stream.py:66-77): per channel d over
// the block's tokens, P = softmax_t(raw_k), z = logsumexp, C = P^T V;
//   dP[t][d] = sum_e dC[d][e] v[t][e],  dv[t][e] += sum_d P[t][d] dC[d][e],
//   d raw_k[t][d] = P (dP - sum_t P dP + dz), with sum_t P dP = sum_e dC C.
// One 512-thread workgroup per (block, batch, head); wave w owns tokens
// [32 w, 32 w + 32). Both products run on v_mfma_f32_32x32x16_bf16 (m = t):
// dP with A = the wave's v rows, B = dC rows [d][e]; dv with A = P rows
// (rebuilt from raw_k and the column statistics), B = dC^T rows [e][d].
constexpr int kWbWaves = 8;

template <int D>
struct WriterBwdSmem {
  bf16_t dc[D][D + 8];          // dC [d][e]
  bf16_t dct[D][D + 8];         // dC^T [e][d]
  float stat[3][D];             // max, 1 / Z, sum_e dC C (+ dz folded into the third)
  float red[kWbWaves][D];
  float red2[kWbWaves][D];      // sum_e dC C partials
};

template <int D>
__global__ __launch_bounds__(kWbWaves * 64) void writer_bwd_kernel(MemBwdParams p) {
  constexpr int KK = D / 16, DT = D / 32, NT = kWbWaves * 64;
  __shared__ WriterBwdSmem<D> sm;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int f = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const int tok0 = f * p.ft;
  const float* dcg = p.dc + ((size_t)bh * p.v_max + f) * D * D;               // dC^T [e][d]
  const bf16_t* c = p.bank + ((size_t)bh * p.fine_cap + f) * D * D;           // C^T [e][d]
  const float* dzf = p.dz + ((size_t)bh * p.v_max + f) * D;
  // ---- stage dC^T (as is) and dC (transposed), bf16; zero when the value
  // matrices are not this writer's (only its z path remains)
  for (int i = tid; i < D * D; i += NT) {
    const int e = i / D, d = i % D;
    const bf16_t v = p.values_external ? (bf16_t)0 : f2bf(dcg[i]);
    sm.dct[e][d] = v;
    sm.dc[d][e] = v;
  }
  // ---- column statistics over the 256 tokens: thread (d, token group) keeps
  // its TPG column values in registers (one read of raw_k); the row term
  // sum_e dC C is split over the same groups (EPG channels e each)
  {
    constexpr int TG = NT / D, TPG = 256 / TG, EPG = D / TG;
    const int d = tid % D, tg = tid / D;
    const bf16_t* col = p.raw_k.p + b * p.raw_k.sb + h * p.raw_k.sh + d;
    float xv[TPG];
#pragma unroll
    for (int i = 0; i < TPG; ++i) xv[i] = bf2f(col[(int64_t)(tok0 + tg * TPG + i) * p.raw_k.st]);
    float sdc = 0.0f;
    if (!p.values_external) {
#pragma unroll 4
      for (int e = tg * EPG; e < (tg + 1) * EPG; ++e)
        sdc = fmaf(dcg[(size_t)e * D + d], bf2f(c[(size_t)e * D + d]), sdc);
    }
    float m = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < TPG; ++i) m = fmaxf(m, xv[i]);
    sm.red[tg][d] = m;
    sm.red2[tg][d] = sdc;
    __syncthreads();
    if (tg == 0) {
      for (int i = 1; i < TG; ++i) m = fmaxf(m, sm.red[i][d]);
      sm.stat[0][d] = m;
    }
    __syncthreads();
    m = sm.stat[0][d];
    float z = 0.0f;
#pragma unroll
    for (int i = 0; i < TPG; ++i) z += __expf(xv[i] - m);
    sm.red[tg][d] = z;                         // the max partials were read before the barrier
    __syncthreads();
    if (tg == 0) {
      for (int i = 1; i < TG; ++i) z += sm.red[i][d];
      sm.stat[1][d] = 1.0f / z;
      float sd = 0.0f;
      for (int i = 0; i < TG; ++i) sd += sm.red2[i][d];
      sm.stat[2][d] = sd - dzf[d];             // dk = P (dP - stat2)
    }
    __syncthreads();
  }
  // ---- A operands of the wave's 32 tokens: v rows and P rows (row li)
  const int t_row = tok0 + 32 * w + li;
  const bf16_t* vrow = p.v.p + b * p.v.sb + (int64_t)t_row * p.v.st + h * p.v.sh;
  const bf16_t* krow = p.raw_k.p + b * p.raw_k.sb + (int64_t)t_row * p.raw_k.st + h * p.raw_k.sh;
  bf16x8 va[KK], pa[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    const int d0 = 16 * kk + 8 * hl;
    va[kk] = as_bf16x8(*(const uint4*)(vrow + d0));
    const uint4 ku = *(const uint4*)(krow + d0);
    const uint32_t kw[4] = {ku.x, ku.y, ku.z, ku.w};
    uint32_t pk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = d0 + 2 * j;
      const float k0 = __uint_as_float(kw[j] << 16), k1 = __uint_as_float(kw[j] & 0xFFFF0000u);
      pk[j] = pack_bf16x2(__expf(k0 - sm.stat[0][d]) * sm.stat[1][d],
                          __expf(k1 - sm.stat[0][d + 1]) * sm.stat[1][d + 1]);
    }
    pa[kk] = as_bf16x8(make_uint4(pk[0], pk[1], pk[2], pk[3]));
  }
  // ---- d raw_k: dP[t][d] (accumulator: lane = d column, rows t_i)
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    floatx16 dp;
#pragma unroll
    for (int i = 0; i < 16; ++i) dp[i] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          va[kk], as_bf16x8(*(const uint4*)&sm.dc[32 * t + li][16 * kk + 8 * hl]), dp, 0, 0, 0);
    const int d = 32 * t + li;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = tok0 + 32 * w + 8 * (i / 4) + 4 * hl + (i % 4);
      const size_t row = ((size_t)b * p.T + tok) * p.H + h;
      const float kv = bf2f(p.raw_k.p[b * p.raw_k.sb + (int64_t)tok * p.raw_k.st + h * p.raw_k.sh + d]);
      const float pr = __expf(kv - sm.stat[0][d]) * sm.stat[1][d];
      const float extra = p.dk_extra ? p.dk_extra[row * D + d] : 0.0f;
      p.draw_k[row * D + d] = f2bf(pr * (dp[i] - sm.stat[2][d]) + extra);
    }
  }
  // ---- dv[t][e] += sum_d P[t][d] dC[d][e] (accumulator: lane = e column)
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          pa[kk], as_bf16x8(*(const uint4*)&sm.dct[32 * t + li][16 * kk + 8 * hl]), acc, 0, 0, 0);
    const int e = 32 * t + li;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = tok0 + 32 * w + 8 * (i / 4) + 4 * hl + (i % 4);
      p.dv[(((size_t)b * p.T + tok) * p.H + h) * D + e] += acc[i];
    }
  }
}

// d raw_q = fusion part + h (dh - sum_d h dh) (softmax adjoint); dv -> bf16;
// d raw_k of tokens no block covers = 0. Thread per channel, row per wave.
template <int D>
__global__ __launch_bounds__(kThreads) void finish_bwd_kernel(MemBwdParams p) {
  constexpr int PER = D / 64;
  const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int rows = p.B * p.T * p.H;
  if (row >= rows) return;
  const int t = (row / p.H) % p.T;
  const int lag = p.keep / p.ft;
  const bool hist = tile_visible(t / p.ft, lag) > 0;
  float hv[PER], dh[PER], s = 0.0f;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int d = lane + 64 * k;
    hv[k] = bf2f(p.h[(size_t)row * D + d]);
    dh[k] = hist ? p.dh[(size_t)row * D + d] : 0.0f;
    s += hv[k] * dh[k];
  }
  s = wave_sum_fold(s);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int d = lane + 64 * k;
    const float g = p.drq_fuse[(size_t)row * D + d] + hv[k] * (dh[k] - s);
    p.draw_q[(size_t)row * D + d] = f2bf(g);
    p.dv_out[(size_t)row * D + d] = f2bf(p.dv[(size_t)row * D + d]);
    if (t >= p.ft * p.v_max) p.draw_k[(size_t)row * D + d] = 0;
  }
}

// The same with eight channels per lane (D / 8 lanes per row, 16-byte loads
// and stores); launch_mem_bwd_writer picks it when every row pointer is 16-byte
// aligned.
template <int D>
__global__ __launch_bounds__(kThreads) void finish_bwd_vec_kernel(MemBwdParams p) {
  constexpr int LPR = D / 8, RPB = kThreads / LPR;
  const int tid = threadIdx.x;
  const int rows = p.B * p.T * p.H;
  const int row = blockIdx.x * RPB + tid / LPR;
  const bool live = row < rows;
  const size_t rr = live ? row : rows - 1;          // the row sum needs every lane
  const int e0 = 8 * (tid % LPR);
  const int t = (int)((rr / p.H) % p.T);
  const bool hist = tile_visible(t / p.ft, p.keep / p.ft) > 0;
  float hv[8], dh[8], s = 0.0f;
  load_bf8(p.h + rr * D + e0, hv);
  if (hist) {
    const float4 d0 = *(const float4*)(p.dh + rr * D + e0);
    const float4 d1 = *(const float4*)(p.dh + rr * D + e0 + 4);
    dh[0] = d0.x; dh[1] = d0.y; dh[2] = d0.z; dh[3] = d0.w;
    dh[4] = d1.x; dh[5] = d1.y; dh[6] = d1.z; dh[7] = d1.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) dh[j] = 0.0f;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) s += hv[j] * dh[j];
  s = row_sum<LPR>(s);
  if (!live) return;
  const float4 q0 = *(const float4*)(p.drq_fuse + rr * D + e0);
  const float4 q1 = *(const float4*)(p.drq_fuse + rr * D + e0 + 4);
  const float4 v0 = *(const float4*)(p.dv + rr * D + e0);
  const float4 v1 = *(const float4*)(p.dv + rr * D + e0 + 4);
  const float dq[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  const float dv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
  float g[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) g[j] = dq[j] + hv[j] * (dh[j] - s);
  store_bf8(p.draw_q + rr * D + e0, g);
  store_bf8(p.dv_out + rr * D + e0, dv);
  if (t >= p.ft * p.v_max) *(uint4*)(p.draw_k + rr * D + e0) = make_uint4(0, 0, 0, 0);
}

}  // namespace

// The larger of the two kernels' grids (d alpha partials to allocate).
int fuse_bwd_workgroups(int T, int B, int H) {
  return ((T + kFuseChunk - 1) / kFuseChunk) * B * H;
}

hipError_t launch_fuse_bwd(const TrainBwdParams& p, int head_dim, hipStream_t s) {
  // 16-byte rows for the vector kernel: aligned bases, bf16 strides in whole
  // 8-element chunks (the fp32 and internal buffers are [rows][D] from aligned
  // allocations)
  auto al = [](const void* q) { return q == nullptr || ((uintptr_t)q & 15) == 0; };
  const bool vec = al(p.grad) && al(p.rq.p) && al(p.local) && al(p.coarse) && al(p.fine) &&
                   al(p.dlocal) && al(p.h) && al(p.dcoarse) && al(p.dnum) && al(p.drq) &&
                   p.g_sb % 8 == 0 && p.g_st % 8 == 0 && p.g_sh % 8 == 0 && p.rq.sb % 8 == 0 &&
                   p.rq.st % 8 == 0 && p.rq.sh % 8 == 0;
  const int chunk = vec ? kFuseVecChunk : kFuseChunk;
  const int groups = ((p.T + chunk - 1) / chunk) * p.B * p.H;
  const dim3 grid((unsigned)groups);
  if (head_dim == 128) {
    if (vec) hipLaunchKernelGGL(fuse_bwd_vec_kernel<128>, grid, dim3(kThreads), 0, s, p);
    else hipLaunchKernelGGL(fuse_bwd_kernel<128>, grid, dim3(kThreads), 0, s, p);
  } else if (head_dim == 64) {
    if (vec) hipLaunchKernelGGL(fuse_bwd_vec_kernel<64>, grid, dim3(kThreads), 0, s, p);
    else hipLaunchKernelGGL(fuse_bwd_kernel<64>, grid, dim3(kThreads), 0, s, p);
  } else {
    return hipErrorInvalidValue;
  }
  if (p.dalpha_parts)
    hipLaunchKernelGGL(dalpha_kernel, dim3(1), dim3(256), 0, s, p.dalpha_parts, groups, p.dalpha);
  return hipGetLastError();
}

hipError_t launch_attn_bwd(const AttnBwdParams& p, int head_dim, hipStream_t s) {
  if (p.T <= 0) return hipSuccess;
  if (p.ft != kFt || p.keep != kKeep) return hipErrorInvalidValue;
  auto rows_grid = [&](int rows) {
    return dim3((unsigned)(((p.T + rows - 1) / rows) * p.B * p.H));
  };
  if (head_dim == 128) {
    hipLaunchKernelGGL(attn_bwd_dq_kernel<128>, rows_grid(kDqWaves<128> * 32),
                       dim3(kDqThreads<128>), 0, s, p);
    hipLaunchKernelGGL(attn_bwd_dkv_kernel<128>, rows_grid(kDkvWaves<128> * 32),
                       dim3(kDkvThreads<128>), 0, s, p);
  } else if (head_dim == 64) {
    hipLaunchKernelGGL(attn_bwd_dq_kernel<64>, rows_grid(kDqWaves<64> * 32),
                       dim3(kDqThreads<64>), 0, s, p);
    hipLaunchKernelGGL(attn_bwd_dkv_kernel<64>, rows_grid(kDkvWaves<64> * 32),
                       dim3(kDkvThreads<64>), 0, s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_mem_bwd_read(const MemBwdParams& p, int head_dim, hipStream_t s) {
  const int BH = p.B * p.H;
  const int n_tiles = (p.T + p.ft - 1) / p.ft;
  // read_bwd keeps the tile's page adjoints in LDS: at most 64 pages.
  if (p.group != 8 || p.ft != 256 || p.v_max / p.group + 1 > 64) return hipErrorInvalidValue;
  if (p.v_max <= 0) return hipSuccess;
  const int lag = p.keep / p.ft;
  const int dc_groups = (std::max(n_tiles - lag - 1, 1) + kObTiles - 1) / kObTiles;
  const int dg_groups = (p.group + kObTilesG - 1) / kObTilesG;
#define TAO_MEM_BWD_READ(D_)                                                                 \
  do {                                                                                       \
    const int blocks = (p.T + kRbQ - 1) / kRbQ;                                              \
    hipLaunchKernelGGL(read_bwd_kernel<D_>, dim3((unsigned)(blocks * BH)),                   \
                       dim3(kRbWaves * 64), 0, s, p);                                        \
    if (p.coarse_values && p.coarse_count > 0) {                                             \
      hipLaunchKernelGGL((outer_bwd_kernel<D_, 1>),                                          \
                         dim3((unsigned)(p.coarse_count * dg_groups * BH)), dim3(kThreads),  \
                         0, s, p, 1);                                                        \
      hipLaunchKernelGGL(coarse_page_bwd_kernel<D_>, dim3((unsigned)(p.coarse_count * BH)),  \
                         dim3(kThreads), 0, s, p);                                           \
    }                                                                                        \
    hipLaunchKernelGGL((outer_bwd_kernel<D_, kObFines<D_>>),                                 \
                       dim3((unsigned)(((p.v_max + kObFines<D_> - 1) / kObFines<D_>) *       \
                                       dc_groups * BH)),                                     \
                       dim3(kThreads), 0, s, p, 0);                                          \
    hipLaunchKernelGGL(page_bwd_kernel<D_>, dim3((unsigned)(n_tiles * BH)), dim3(D_), 0, s,  \
                       p);                                                                   \
    if (p.v_max / p.group > 0)                                                               \
      hipLaunchKernelGGL(zpage_bwd_kernel<D_>, dim3((unsigned)((p.v_max / p.group) * BH)),   \
                         dim3(D_), 0, s, p);                                                 \
  } while (0)
  if (head_dim == 128)
    TAO_MEM_BWD_READ(128);
  else if (head_dim == 64)
    TAO_MEM_BWD_READ(64);
  else
    return hipErrorInvalidValue;
#undef TAO_MEM_BWD_READ
  return hipGetLastError();
}

hipError_t launch_mem_bwd_writer(const MemBwdParams& p, int head_dim, hipStream_t s) {
  const int BH = p.B * p.H;
  auto al = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  const bool fin_vec = al(p.h) && al(p.dh) && al(p.drq_fuse) && al(p.dv) && al(p.draw_q) &&
                       al(p.dv_out) && al(p.draw_k);
#define TAO_MEM_BWD_WRITER(D_)                                                               \
  do {                                                                                       \
    if (p.v_max > 0)                                                                         \
      hipLaunchKernelGGL(writer_bwd_kernel<D_>, dim3((unsigned)(p.v_max * BH)),              \
                         dim3(kWbWaves * 64), 0, s, p);                                      \
    const int rows = p.B * p.T * p.H;                                                        \
    constexpr int vrows = kThreads / (D_ / 8);                                               \
    if (fin_vec)                                                                             \
      hipLaunchKernelGGL(finish_bwd_vec_kernel<D_>, dim3((unsigned)((rows + vrows - 1) / vrows)),\
                         dim3(kThreads), 0, s, p);                                           \
    else                                                                                     \
      hipLaunchKernelGGL(finish_bwd_kernel<D_>,                                              \
                         dim3((unsigned)((rows + kThreads / 64 - 1) / (kThreads / 64))),     \
                         dim3(kThreads), 0, s, p);                                           \
  } while (0)
  if (head_dim == 128)
    TAO_MEM_BWD_WRITER(128);
  else if (head_dim == 64)
    TAO_MEM_BWD_WRITER(64);
  else
    return hipErrorInvalidValue;
#undef TAO_MEM_BWD_WRITER
  return hipGetLastError();
}

}  // namespace tao
