// Routing refresh for gfx950: one workgroup per (batch, head).
//
// Restates tao_stream.py:310-357 with _topk_oldest (:50-53):
//   h    = r(softmax_D(raw_q))                 (anchor query row)
//   hv_p = r(h * pw[p])                        (page weights of the epoch)
//   page mass = r(sum_D hv_p) over completed pages; stable top-`coarse`
//   pages (descending, lowest index wins ties), re-sorted ascending;
//   candidates = 8 fines of each chosen page + every pending fine;
//   mass_j = r(sum_D r(hv_page(j) * sw_j)); stable top-M candidates kept in
//   score order.
// Every fp32 sum uses the butterfly order of the oracle, so selected ids are
// bit-identical to the oracle's. Sorting: 64-bit keys
// (monotone bf16 score << 32 | ~index) in an LDS bitonic network.
#include "tao_launch.h"
#include "tao_common.h"

namespace tao {
namespace {

constexpr int kMaxSort = 2048;   // pages or candidates per head

template <int D>
struct RouteSmem {
  float h[D];
  unsigned long long keys[kMaxSort];
  int cand_id[kMaxSort];
  int cand_page[kMaxSort];
  int chosen[kMaxSort / 8];
};

__device__ void bitonic_desc(unsigned long long* keys, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += kThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const unsigned long long a = keys[i], b = keys[ixj];
          const bool first_half_desc = (i & k) == 0;
          if (first_half_desc ? (a < b) : (a > b)) { keys[i] = b; keys[ixj] = a; }
        }
      }
      __syncthreads();
    }
  }
}

TAO_DEV unsigned long long score_key(float score_bf, int index) {
  const uint32_t hi = bf16_order_key(f2bf(score_bf));
  return ((unsigned long long)hi << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)index);
}

TAO_DEV int key_index(unsigned long long key) {
  return (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
}

// r(sum_D r(h * pw[page]) * (sw row or 1)) computed by one wave.
template <int D>
TAO_DEV float wave_mass(const float* h, const bf16_t* pw_row, const bf16_t* sw_row, int lane) {
  constexpr int PER = D / 64;
  float v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int d = lane + 64 * k;
    float hv = rbf(h[d] * bf2f(pw_row[d]));
    v[k] = sw_row ? rbf(hv * bf2f(sw_row[d])) : hv;
  }
  float s = v[0];
#pragma unroll
  for (int k = 1; k < PER; ++k) s += v[k];
  return rbf(wave_sum_fold(s));
}

template <int D>
__global__ __launch_bounds__(kThreads) void route_kernel(RouteParams p) {
  __shared__ RouteSmem<D> sm;
  constexpr int PER = D / 64;
  const int bh = blockIdx.x;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bf16_t* pw = p.pw + (size_t)bh * p.page_cap * D;
  const bf16_t* sw = p.sw + (size_t)bh * p.fine_cap * D;

  if (wave == 0) {
    const bf16_t* rq = p.rq + b * p.rq_sb + h * p.rq_sh;
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
    for (int k = 0; k < PER; ++k) sm.h[lane + 64 * k] = rbf(e[k] / s);
  }
  __syncthreads();

  // ---- coarse pages
  const int K = p.completed;
  if (p.coarse > 0) {
    int np = 1;
    while (np < K) np <<= 1;
    for (int i = tid; i < np; i += kThreads) sm.keys[i] = 0ull;
    __syncthreads();
    for (int page = wave; page < K; page += kThreads / 64) {
      const float mass = wave_mass<D>(sm.h, pw + (size_t)page * D, nullptr, lane);
      if (lane == 0) sm.keys[page] = score_key(mass, page);
    }
    __syncthreads();
    bitonic_desc(sm.keys, np);
    // chosen pages ascending: rank among the top `coarse`.
    if (tid < p.coarse) {
      const int mine = key_index(sm.keys[tid]);
      int rank = 0;
      for (int j = 0; j < p.coarse; ++j) rank += key_index(sm.keys[j]) < mine;
      sm.chosen[rank] = mine;
    }
    __syncthreads();
  }

  // ---- candidates
  const int group = p.group;
  const int E = group * p.coarse + p.pending;
  for (int j = tid; j < E; j += kThreads) {
    int page, id;
    if (j < group * p.coarse) {
      page = sm.chosen[j / group];
      id = page * group + j % group;
    } else {
      page = K;
      id = K * group + (j - group * p.coarse);
    }
    sm.cand_page[j] = page;
    sm.cand_id[j] = id;
  }
  int ne = 1;
  while (ne < E) ne <<= 1;
  __syncthreads();
  for (int i = tid; i < ne; i += kThreads) sm.keys[i] = 0ull;
  __syncthreads();
  for (int j = wave; j < E; j += kThreads / 64) {
    const float mass = wave_mass<D>(sm.h, pw + (size_t)sm.cand_page[j] * D,
                                    sw + (size_t)sm.cand_id[j] * D, lane);
    if (lane == 0) sm.keys[j] = score_key(mass, j);
  }
  __syncthreads();
  bitonic_desc(sm.keys, ne);
  for (int m = tid; m < p.selected; m += kThreads)
    p.sel[(size_t)bh * p.sel_cap + m] = sm.cand_id[key_index(sm.keys[m])];
  for (int i = tid; i < p.coarse; i += kThreads)
    p.chosen[(size_t)bh * p.chosen_cap + i] = sm.chosen[i];
  if (bh == 0 && tid == 0) p.header[1] = p.selected;
}

}  // namespace

hipError_t launch_route(const RouteParams& p, int head_dim, hipStream_t s) {
  if (p.completed > kMaxSort || p.group * p.coarse + p.pending > kMaxSort)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)(p.B * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(route_kernel<128>, grid, dim3(kThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(route_kernel<64>, grid, dim3(kThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace tao
