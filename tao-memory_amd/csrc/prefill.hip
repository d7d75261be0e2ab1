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
// read_tiles_kernel: one workgroup per (tile of <= 32 queries sharing one
// route, batch, head). For each selected fine m:
//   ch[q][d] = r(r(h_q[d] * pw[page][d]) * sw[fine][d])   (LDS, bf16)
//   num[q][e] += sum_d ch[q][d] * C[d][e]                  v_mfma_f32_32x32x16_bf16
// with the B operand C^T[e][d] read straight from the bank (d contiguous)
// and prefetched one fine ahead. den = r(sum_m r(sum_d ch)) in butterfly
// order, fine = r(r(num)/den), then the fusion epilogue with the local
// attention output. Tiles of one head share blockIdx % 8 (XCD) when B*H is
// a multiple of 8, so a head's bank stays in one XCD's L2.
#include "tao_launch.h"
#include "tao_common.h"
#include "tao_fusion.h"

namespace tao {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kTileQ = 32;
constexpr int kMaxM = 128;

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
  int width = 1;
  while (width * 64 < P) width <<= 1;
  const bf16_t* pzg = p.page_z + (size_t)bh * p.page_cap * D;
  bf16_t* state_pw = p.page_w + (size_t)bh * p.page_cap * D;
  for (int d = wave; d < D; d += kThreads / 64) {
    float x[32];
    float m = -__builtin_inff();
    for (int k = 0; k < width; ++k) {
      const int pg = lane + 64 * k;
      x[k] = pg < P ? (pg == K ? pend_pz[d] : bf2f(pzg[(size_t)pg * D + d])) : -__builtin_inff();
      m = fmaxf(m, x[k]);
    }
    m = wave_max(m);
    float e[32];
    for (int k = 0; k < width; ++k) e[k] = (lane + 64 * k) < P ? exp_cr(x[k] - m) : 0.0f;
    for (int w = width / 2; w >= 1; w >>= 1)
      for (int k = 0; k < w; ++k) e[k] += e[k + w];
    const float total = wave_sum_fold(e[0]);
    for (int k = 0; k < width; ++k) {
      const int pg = lane + 64 * k;
      if (pg < P) {
        const bf16_t w = f2bf(exp_cr(x[k] - m) / total);
        pw[(size_t)pg * D + d] = w;
        if (last) state_pw[(size_t)pg * D + d] = w;
      }
    }
  }
}

template <int D>
__global__ __launch_bounds__(kThreads) void read_tiles_kernel(ReadTilesParams p) {
  constexpr int PER = D / 64, KK = D / 16, ET = D / 32;
  __shared__ float hq[kTileQ][D];
  __shared__ bf16_t chs[2][kTileQ][D + 8];
  __shared__ float chsum[kTileQ][kMaxM];
  __shared__ int ids[kMaxM];
  __shared__ float den[kTileQ];
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int tile = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int64_t* desc = p.tiles + 8 * tile;
  const int q_first = (int)desc[0], nq = (int)desc[1], slot = (int)desc[2];
  const int M = (int)desc[3], erel = (int)desc[4], sw_split = (int)desc[5];
  const int fine_on = (int)desc[6];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;

  if (!fine_on) {
    for (int i = tid; i < nq * (D / 8); i += kThreads) {
      const int q = i / (D / 8), c = i % (D / 8);
      const int t = q_first + q;
      *(uint4*)(p.out + b * p.out_sb + (int64_t)t * p.out_st + h * p.out_sh + c * 8) =
          *(const uint4*)(p.local + (((size_t)b * p.T + t) * p.H + h) * D + c * 8);
    }
    return;
  }
  const int32_t* sel = p.sel_pool + ((size_t)slot * BH + bh) * p.sel_cap;
  for (int m = tid; m < M; m += kThreads) ids[m] = sel[m];
  // h = r(softmax_D(raw_q)) of the tile's queries; wave w owns q = w + 4j,
  // all of its rows are loaded before any reduction.
  constexpr int QPW = kTileQ / (kThreads / 64);
  float xr[QPW][PER];
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
    const int q = wave + 4 * j;
    const bf16_t* rq = p.rq.p + b * p.rq.sb + (int64_t)(q_first + min(q, nq - 1)) * p.rq.st +
                       h * p.rq.sh;
#pragma unroll
    for (int k = 0; k < PER; ++k) xr[j][k] = bf2f(rq[lane + 64 * k]);
  }
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
    const int q = wave + 4 * j;
    float mx = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < PER; ++k) mx = fmaxf(mx, xr[j][k]);
    mx = wave_max(mx);
    float e[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) e[k] = exp_cr(xr[j][k] - mx);
    float s = e[0];
#pragma unroll
    for (int k = 1; k < PER; ++k) s += e[k];
    s = wave_sum_fold(s);
#pragma unroll
    for (int k = 0; k < PER; ++k) hq[q][lane + 64 * k] = q < nq ? rbf(e[k] / s) : 0.0f;
  }
  __syncthreads();
  const bf16_t* bank = p.bank + (size_t)bh * p.fine_cap * D * D;
  const bf16_t* pw_base = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
  const bf16_t* psw_base = p.psw_pool ? p.psw_pool + ((size_t)erel * BH + bh) * 8 * D : nullptr;
  const bf16_t* sw_base = p.sw + (size_t)bh * p.fine_cap * D;
  const int e_row = 32 * wave + li;          // C^T row this lane feeds (wave < ET)

  // Operands of fine `id`: C^T rows (waves < ET), page-weight and
  // segment-weight channels of this lane.
  auto fetch = [&](int id, uint4* c, float* pwv, float* swv) {
    if (wave < ET) {
      const bf16_t* crow = bank + ((size_t)id * D + e_row) * D;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) c[kk] = *(const uint4*)(crow + 16 * kk + 8 * hl);
    }
    const bf16_t* pw = pw_base + (size_t)(id / p.group) * D;
    const bf16_t* sw = id < sw_split ? sw_base + (size_t)id * D
                                     : psw_base + (size_t)(id - sw_split) * D;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      pwv[k] = bf2f(pw[lane + 64 * k]);
      swv[k] = bf2f(sw[lane + 64 * k]);
    }
  };

  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  uint4 creg[KK], cnext[KK];
  float pwv[PER], swv[PER], pwn[PER], swn[PER];
  fetch(ids[0], creg, pwv, swv);
  for (int m = 0; m < M; ++m) {
    const int buf = m & 1;
    for (int q = wave; q < kTileQ; q += kThreads / 64) {
      float v[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int d = lane + 64 * k;
        v[k] = q < nq ? rbf(rbf(hq[q][d] * pwv[k]) * swv[k]) : 0.0f;
        chs[buf][q][d] = f2bf(v[k]);
      }
      float s = v[0];
#pragma unroll
      for (int k = 1; k < PER; ++k) s += v[k];
      s = wave_sum_fold(s);
      if (lane == 0) chsum[q][m] = rbf(s);
    }
    if (m + 1 < M) fetch(ids[m + 1], cnext, pwn, swn);
    __syncthreads();
    if (wave < ET) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const bf16x8 a = as_bf16x8(*(const uint4*)&chs[buf][li][16 * kk + 8 * hl]);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, as_bf16x8(creg[kk]), acc, 0, 0, 0);
      }
    }
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) creg[kk] = cnext[kk];
#pragma unroll
    for (int k = 0; k < PER; ++k) { pwv[k] = pwn[k]; swv[k] = swn[k]; }
  }
  __syncthreads();
  // den per query: slot m in lane m % 64, position m / 64 (M <= 128).
  for (int q = wave; q < kTileQ; q += kThreads / 64) {
    const float v0 = lane < M ? chsum[q][lane] : 0.0f;
    const float v1 = lane + 64 < M ? chsum[q][lane + 64] : 0.0f;
    const float s = wave_sum_fold(M > 64 ? v0 + v1 : v0);
    if (lane == 0) den[q] = rbf(s);
  }
  __syncthreads();
  if (wave >= ET) return;
  const int e = 32 * wave + li;
  float a[3], bb[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    a[i] = load_param(p.fa, p.f_dtype, h * p.fa_s[0] + e * p.fa_s[1] + i * p.fa_s[2]);
    bb[i] = load_param(p.fb, p.f_dtype, h * p.fb_s[0] + e * p.fb_s[1] + i * p.fb_s[2]);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int q = 8 * (i / 4) + 4 * hl + (i % 4);
    if (q < nq) {
      const int t = q_first + q;
      const float fine = rbf(rbf(acc[i]) / den[q]);
      const float local = bf2f(p.local[(((size_t)b * p.T + t) * p.H + h) * D + e]);
      const float x = bf2f(p.rq.p[b * p.rq.sb + (int64_t)t * p.rq.st + h * p.rq.sh + e]);
      p.out[b * p.out_sb + (int64_t)t * p.out_st + h * p.out_sh + e] =
          fuse_element(x, local, 0.0f, fine, a, bb, p.gain, 0, 1);
    }
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
  const dim3 grid((unsigned)(p.n_tiles * p.B * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(read_tiles_kernel<128>, grid, dim3(kThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(read_tiles_kernel<64>, grid, dim3(kThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace tao
