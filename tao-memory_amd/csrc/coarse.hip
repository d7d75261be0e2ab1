// Coarse value branch for gfx950 (TaoConfig.coarse_index_only = False).
//
// page_coarse_kernel (once per completed page): the page's value matrix is
// the segment-weighted sum of its fine memories (append_fine,
// tao_stream.py:486-499),
//   page_C^T[e][d] = r(sum_s w_s[d] C^T_s[e][d]),  w_s = r(exp(r(z_s - page_z)))
// which is the page's final fine_sw row, so it is built from the bank and
// fine_sw after the seal epilogue.
//
// coarse_fold_kernel (once per page completion, not per token): the coarse
// read of _read_reused (tao_stream.py:299-305) is
//   coarse[e] = sum_p sum_d h[d] cw_p[d] page_C_p[d][e],
//   cw = softmax over the completed pages of page_z,
// linear in h with query-independent weights, so the pages fold into one
// D x D matrix per head, G^T[e][d] = sum_p cw_p[d] page_C^T_p[e][d], and a
// query reads 32/64 KB per head instead of P page matrices. One pass over
// the pages keeps an online softmax per column d (running max, rescaled sum
// and accumulator) and emits G^T(n) for every page count n of a range: the
// prefill pool needs one per page epoch, the decode state the last one.
// The reference rounds cw and h * cw to bf16 before an fp32 contraction;
// the fold keeps both in fp32 (outputs only, within the bf16 tolerance).
#include "tao_launch.h"
#include "tao_common.h"

namespace tao {
namespace {

TAO_DEV void unpack8c(const uint4& u, float out[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

// Thread (row r, chunk c) of a workgroup covers G^T / page_C^T row e0 + r,
// columns [8c, 8c + 8); ROWS rows per workgroup, CHUNKS workgroups per head.
template <int D>
struct CoarseGeo {
  static constexpr int CH = D / 8;
  static constexpr int ROWS = kThreads / CH;
  static constexpr int CHUNKS = D / ROWS;
};

template <int D>
__global__ __launch_bounds__(kThreads) void page_coarse_kernel(PageCoarseParams p) {
  using G = CoarseGeo<D>;
  const int BH = p.B * p.H;
  const int chunk = blockIdx.x % G::CHUNKS;
  const int bh = (blockIdx.x / G::CHUNKS) % BH;
  const int page = p.first_page + blockIdx.x / (G::CHUNKS * BH);
  const int tid = threadIdx.x, c = tid % G::CH, r = tid / G::CH;
  const int e = chunk * G::ROWS + r;
  const bf16_t* bank = p.bank + ((size_t)bh * p.fine_cap + (size_t)page * p.group) * D * D;
  const bf16_t* sw = p.sw + ((size_t)bh * p.fine_cap + (size_t)page * p.group) * D;
  uint4 cv[8], wv[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    cv[s] = *(const uint4*)(bank + ((size_t)s * D + e) * D + c * 8);
    wv[s] = *(const uint4*)(sw + (size_t)s * D + c * 8);
  }
  float acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = 0.0f;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    float cf[8], wf[8];
    unpack8c(cv[s], cf);
    unpack8c(wv[s], wf);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = fmaf(wf[k], cf[k], acc[k]);
  }
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = pack_bf16x2(acc[2 * k], acc[2 * k + 1]);
  *(uint4*)(p.page_c + (((size_t)bh * p.page_cap + page) * D + e) * D + c * 8) =
      make_uint4(o[0], o[1], o[2], o[3]);
}

template <int D>
__global__ __launch_bounds__(kThreads) void coarse_fold_kernel(CoarseFoldParams p) {
  using G = CoarseGeo<D>;
  constexpr int U = 4;   // pages in flight
  const int BH = p.B * p.H;
  const int chunk = blockIdx.x % G::CHUNKS;
  const int bh = blockIdx.x / G::CHUNKS;
  const int tid = threadIdx.x, c = tid % G::CH, r = tid / G::CH;
  const int e = chunk * G::ROWS + r;
  const bf16_t* pz = p.page_z + (size_t)bh * p.page_cap * D + c * 8;
  const bf16_t* pc = p.page_c + (size_t)bh * p.page_cap * D * D + (size_t)e * D + c * 8;
  const int last = p.n_first + p.n_count - 1;
  float m[8], s[8], acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) { m[k] = -__builtin_inff(); s[k] = 0.0f; acc[k] = 0.0f; }
  for (int p0 = 0; p0 < last; p0 += U) {
    uint4 zv[U], cv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int pg = min(p0 + u, last - 1);
      zv[u] = *(const uint4*)(pz + (size_t)pg * D);
      cv[u] = *(const uint4*)(pc + (size_t)pg * D * D);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int pg = p0 + u;
      if (pg < last) {
        float zf[8], cf[8];
        unpack8c(zv[u], zf);
        unpack8c(cv[u], cf);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float mn = fmaxf(m[k], zf[k]);
          const float keep = __expf(m[k] - mn);
          const float w = __expf(zf[k] - mn);
          s[k] = fmaf(s[k], keep, w);
          acc[k] = fmaf(acc[k], keep, w * cf[k]);
          m[k] = mn;
        }
        const int n = pg + 1;   // pages folded so far
        if (n >= p.n_first) {
          const size_t off = ((size_t)(n - p.n_first) * BH + bh) * D * D + (size_t)e * D + c * 8;
          float g[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) g[k] = acc[k] / s[k];
          if (p.out_f32) {
            float* o = (float*)p.out + off;
            *(float4*)o = make_float4(g[0], g[1], g[2], g[3]);
            *(float4*)(o + 4) = make_float4(g[4], g[5], g[6], g[7]);
          } else {
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = pack_bf16x2(g[2 * k], g[2 * k + 1]);
            *(uint4*)((bf16_t*)p.out + off) = make_uint4(o[0], o[1], o[2], o[3]);
          }
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_page_coarse(const PageCoarseParams& p, int head_dim, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  if (p.group != 8 || p.first_page < 0 || p.first_page + p.count > p.page_cap ||
      (p.first_page + p.count) * p.group > p.fine_cap)
    return hipErrorInvalidValue;
  if (head_dim == 128) {
    const dim3 grid((unsigned)(p.count * p.B * p.H * CoarseGeo<128>::CHUNKS));
    hipLaunchKernelGGL(page_coarse_kernel<128>, grid, dim3(kThreads), 0, s, p);
  } else if (head_dim == 64) {
    const dim3 grid((unsigned)(p.count * p.B * p.H * CoarseGeo<64>::CHUNKS));
    hipLaunchKernelGGL(page_coarse_kernel<64>, grid, dim3(kThreads), 0, s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_coarse_fold(const CoarseFoldParams& p, int head_dim, hipStream_t s) {
  if (p.n_count <= 0) return hipSuccess;
  if (p.n_first < 1 || p.n_first + p.n_count - 1 > p.page_cap) return hipErrorInvalidValue;
  if (head_dim == 128) {
    const dim3 grid((unsigned)(p.B * p.H * CoarseGeo<128>::CHUNKS));
    hipLaunchKernelGGL(coarse_fold_kernel<128>, grid, dim3(kThreads), 0, s, p);
  } else if (head_dim == 64) {
    const dim3 grid((unsigned)(p.B * p.H * CoarseGeo<64>::CHUNKS));
    hipLaunchKernelGGL(coarse_fold_kernel<64>, grid, dim3(kThreads), 0, s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace tao
