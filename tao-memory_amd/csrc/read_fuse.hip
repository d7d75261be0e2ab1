// Selected fine read + fusion for a run of queries that share one route.
//
// Restates query_fresh_fine.py:8-75 for multi-token calls and the fusion
// kernels fusion_pointwise.py:10-117 (operator.py:86-97): one workgroup per
// (batch, head, block of kQB queries). For each selected fine m (slot order)
// the workgroup streams C_m once and contracts it with every query's bf16
// channel weights ch[q] = r(r(h_q * pw[page]) * sw[fine]); num accumulates in
// fp32 across slots, den = r(sum_m r(sum_d ch)) in the oracle's butterfly
// order, fine = r(r(num) / den), then the fusion epilogue with the local
// attention output writes the heads.
#include "tao_launch.h"
#include "tao_common.h"
#include "tao_fusion.h"

namespace tao {
namespace {

constexpr int kQB = 16;
constexpr int kMaxSel = 512;

template <int D>
struct ReadSmem {
  float h[kQB][D];
  float ch[kQB][D];
  float red[kThreads / (D / 8)][D];
  float den[kQB];
};

TAO_DEV void unpack8r(const uint4& u, float out[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

template <int D>
__global__ __launch_bounds__(kThreads) void read_fuse_kernel(ReadParams p) {
  __shared__ ReadSmem<D> sm;
  constexpr int CH = D / 8, ROWS = kThreads / CH, RPT = D / ROWS, PER = D / 64;
  const int nqb = (p.count + kQB - 1) / kQB;
  const int bh = blockIdx.x / nqb;
  const int qb = blockIdx.x % nqb;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = tid % CH, r = tid / CH;
  const int q0 = p.first + qb * kQB;
  const int nq = min(kQB, p.first + p.count - q0);
  const int M = p.fine_on ? p.selected : 0;

  // h = r(softmax_D(raw_q)) per query, one wave per query.
  for (int q = wave; q < nq; q += kThreads / 64) {
    const bf16_t* rq = p.rq.p + b * p.rq.sb + (long long)(q0 + q) * p.rq.st + h * p.rq.sh;
    float x[PER], e[PER];
    float top = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < PER; ++k) { x[k] = bf2f(rq[lane + 64 * k]); top = fmaxf(top, x[k]); }
    top = wave_max(top);
#pragma unroll
    for (int k = 0; k < PER; ++k) e[k] = exp_cr(x[k] - top);
    float s = e[0];
#pragma unroll
    for (int k = 1; k < PER; ++k) s += e[k];
    s = wave_sum_fold(s);
#pragma unroll
    for (int k = 0; k < PER; ++k) sm.h[q][lane + 64 * k] = rbf(e[k] / s);
  }
  // Per-slot r(sum_d ch) of the queries this wave owns (q = wave + 4i):
  // slot m sits in lane m % 64 at position m / 64 (M <= 512), the layout of
  // the oracle's butterfly order over slots.
  float den_hi[kQB / 4][8];
  for (int i = 0; i < kQB / 4; ++i)
    for (int k = 0; k < 8; ++k) den_hi[i][k] = 0.0f;

  float acc[kQB][8];
#pragma unroll
  for (int q = 0; q < kQB; ++q)
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[q][k] = 0.0f;

  const bf16_t* bank = p.bank + (size_t)bh * p.fine_cap * D * D;
  for (int m = 0; m < M; ++m) {
    const int id = p.sel[(size_t)bh * p.sel_cap + m];
    const int page = id / p.group;
    const bf16_t* cmat = bank + (size_t)id * D * D;
    uint4 cv[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) cv[i] = *(const uint4*)(cmat + (size_t)(r + i * ROWS) * D + c * 8);
    __syncthreads();   // h ready / previous ch consumed
    const bf16_t* pw = p.pw + ((size_t)bh * p.page_cap + page) * D;
    const bf16_t* sw = p.sw + ((size_t)bh * p.fine_cap + id) * D;
    for (int q = wave; q < kQB; q += kThreads / 64) {
      float part[PER];
      float csum = 0.0f;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int d = lane + 64 * k;
        float ch = 0.0f;
        if (q < nq) ch = rbf(rbf(sm.h[q][d] * bf2f(pw[d])) * bf2f(sw[d]));
        sm.ch[q][d] = ch;
        part[k] = ch;
      }
      csum = part[0];
#pragma unroll
      for (int k = 1; k < PER; ++k) csum += part[k];
      csum = rbf(wave_sum_fold(csum));
      // slot m lives in lane m % 64, in-lane position m / 64.
      const int qi = q / 4;
      if (lane == (m & 63)) den_hi[qi][m >> 6] = csum;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int d = r + i * ROWS;
      float cf[8];
      unpack8r(cv[i], cf);
#pragma unroll
      for (int q = 0; q < kQB; ++q) {
        const float w = sm.ch[q][d];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[q][k] = fmaf(w, cf[k], acc[q][k]);
      }
    }
  }
  // den per query: butterfly over slots (lane m%64, in-lane index m/64).
  if (M > 0) {
    int width = 1;
    while (width * 64 < M) width <<= 1;
    for (int q = wave; q < kQB; q += kThreads / 64) {
      const int qi = q / 4;
      float v[8];
      for (int k = 0; k < 8; ++k) v[k] = den_hi[qi][k];
      for (int w = width / 2; w >= 1; w >>= 1)
        for (int k = 0; k < w; ++k) v[k] += v[k + w];
      const float den = rbf(wave_sum_fold(v[0]));
      if (lane == 0) sm.den[q] = den;
    }
  }
  // Reduce acc over row groups, one query at a time, then fuse and store.
  for (int q = 0; q < nq; ++q) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 8; ++k) sm.red[r][c * 8 + k] = acc[q][k];
    __syncthreads();
    if (tid < D) {
      const int t = q0 + q;
      float num = 0.0f;
      for (int rr = 0; rr < ROWS; ++rr) num += sm.red[rr][tid];
      const float local = bf2f(p.local[(((size_t)b * p.T + t) * p.H + h) * D + tid]);
      bf16_t result;
      if (p.fine_on || p.coarse_on) {
        const float fine = M > 0 ? rbf(rbf(num) / sm.den[q]) : 0.0f;
        const float x = bf2f(p.rq.p[b * p.rq.sb + (long long)t * p.rq.st + h * p.rq.sh + tid]);
        float a[3], bb[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          a[i] = load_param(p.fa, p.f_dtype, h * p.fa_s[0] + tid * p.fa_s[1] + i * p.fa_s[2]);
          bb[i] = load_param(p.fb, p.f_dtype, h * p.fb_s[0] + tid * p.fb_s[1] + i * p.fb_s[2]);
        }
        result = fuse_element(x, local, 0.0f, fine, a, bb, p.gain, p.coarse_on, p.fine_on);
      } else {
        result = f2bf(local);
      }
      p.out[b * p.out_sb + (long long)t * p.out_st + h * p.out_sh + tid] = result;
    }
  }
}

}  // namespace

hipError_t launch_read_fuse(const ReadParams& p, int head_dim, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  if (p.selected > kMaxSel) return hipErrorInvalidValue;
  const int nqb = (p.count + kQB - 1) / kQB;
  const dim3 grid((unsigned)(p.B * p.H * nqb));
  if (head_dim == 128)
    hipLaunchKernelGGL(read_fuse_kernel<128>, grid, dim3(kThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(read_fuse_kernel<64>, grid, dim3(kThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace tao
