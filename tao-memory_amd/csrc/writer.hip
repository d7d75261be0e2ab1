// Softmax fine writer and seal epilogue for gfx950.
//
// writer_kernel: one workgroup per (block, batch, head). Restates _seal's
// softmax branch (tao_stream.py:66-77) for a 256-token block:
//   per channel d: m = max_t k, e = r(exp(r(k - m))), Z = r(sum_t e),
//   P = r(e / Z), z = r(m + r(log Z)); C = r(P^T V) with fp32 accumulation.
// raw_k and V are staged transposed in LDS ([channel][token], token
// contiguous) so both MFMA operands are 16-byte LDS reads; C^T = V^T P runs
// on v_mfma_f32_32x32x16_bf16 (each wave owns 32 rows of C^T). The bank keeps
// C^T[e][d] so the contraction index d is contiguous for every reader. The
// token sum uses
// the oracle's order: four 64-token quarters summed sequentially, then
// (q0+q1)+(q2+q3). C goes straight into its bank slot: no repack.
//
// epilogue_kernel: one workgroup per (batch, head) after sealing fine `slot`
// (append_fine, tao_stream.py:477-501, plus the pending summary :277-290
// and the seal-epoch memo :399-416): page descriptor
// pz = logsumexp over the slot's group (torch's bf16 composite), segment
// weights sw = r(exp(r(z - pz))) of the group's fines, and page weights
// pw = r(softmax over pages) for every current page.
#include "tao_launch.h"
#include "tao_common.h"

namespace tao {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBlock = 256;                 // tokens per fine block
constexpr int kRowPad = kBlock + 8;         // LDS row stride in bf16 (528 B)

template <int D>
struct WriterSmem {
  bf16_t kt[D][kRowPad];   // raw keys, then probabilities P^T
  bf16_t vt[D][kRowPad];   // values transposed
  float part[4][D];
  float top[D];
  float total[D];
};

TAO_DEV const bf16_t* token_row(const WriterParams& p, int b, int h, long long pos,
                                const TokView& tv, const bf16_t* ring, int D) {
  if (pos >= p.new_base) {
    const long long t = pos - p.new_base;
    return tv.p + b * tv.sb + t * tv.st + h * tv.sh;
  }
  const int slot = (int)(pos % p.L);
  return ring + (((size_t)b * p.L + slot) * p.H + h) * D;
}

constexpr int kWriterThreads = 512;   // 8 waves

// Stage raw_k and V of one block transposed into LDS ([channel][token]).
// Every global load of the block is issued before the first LDS write; job
// -> (channel chunk c, token pair): 128 consecutive jobs share c, so a
// half-wave's transposing 4-byte writes fill consecutive words of one row.
template <int D>
__device__ void stage_block(const WriterParams& p, int b, int h, long long start,
                            bf16_t (*kt)[kRowPad], bf16_t (*vt)[kRowPad]) {
  constexpr int CH = D / 8;
  constexpr int JOBS = (kBlock / 2) * CH / kWriterThreads;   // token pairs per thread
  uint4 ka[JOBS], kb[JOBS], va[JOBS], vb[JOBS];
#pragma unroll
  for (int j = 0; j < JOBS; ++j) {
    const int job = threadIdx.x + j * kWriterThreads;
    const int c = job / (kBlock / 2), t0 = 2 * (job % (kBlock / 2));
    ka[j] = *(const uint4*)(token_row(p, b, h, start + t0, p.rk, p.ring_raw, D) + c * 8);
    kb[j] = *(const uint4*)(token_row(p, b, h, start + t0 + 1, p.rk, p.ring_raw, D) + c * 8);
    va[j] = *(const uint4*)(token_row(p, b, h, start + t0, p.v, p.ring_v, D) + c * 8);
    vb[j] = *(const uint4*)(token_row(p, b, h, start + t0 + 1, p.v, p.ring_v, D) + c * 8);
  }
#pragma unroll
  for (int j = 0; j < JOBS; ++j) {
    const int job = threadIdx.x + j * kWriterThreads;
    const int c = job / (kBlock / 2), t0 = 2 * (job % (kBlock / 2));
    const uint32_t wa[4] = {ka[j].x, ka[j].y, ka[j].z, ka[j].w};
    const uint32_t wb[4] = {kb[j].x, kb[j].y, kb[j].z, kb[j].w};
    const uint32_t xa[4] = {va[j].x, va[j].y, va[j].z, va[j].w};
    const uint32_t xb[4] = {vb[j].x, vb[j].y, vb[j].z, vb[j].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *(uint32_t*)&kt[c * 8 + 2 * i][t0] = (wa[i] & 0xFFFFu) | (wb[i] << 16);
      *(uint32_t*)&kt[c * 8 + 2 * i + 1][t0] = (wa[i] >> 16) | (wb[i] & 0xFFFF0000u);
      *(uint32_t*)&vt[c * 8 + 2 * i][t0] = (xa[i] & 0xFFFFu) | (xb[i] << 16);
      *(uint32_t*)&vt[c * 8 + 2 * i + 1][t0] = (xa[i] >> 16) | (xb[i] & 0xFFFF0000u);
    }
  }
}

template <int D>
__global__ __launch_bounds__(kWriterThreads) void writer_kernel(WriterParams p) {
  __shared__ WriterSmem<D> sm;
  const int bh = blockIdx.x % (p.B * p.H);
  const int blk = blockIdx.x / (p.B * p.H);
  const int b = bh / p.H, h = bh % p.H;
  const long long start = p.starts[blk];
  const int slot = p.first_slot + blk;
  const int tid = threadIdx.x;

  stage_block<D>(p, b, h, start, sm.kt, sm.vt);
  __syncthreads();

  // ---- column softmax: jobs (channel, quarter of 64 tokens)
  constexpr int QT = kBlock / 4;
  for (int job = tid; job < 4 * D; job += kWriterThreads) {
    const int d = job % D, qq = job / D;
    float m = -__builtin_inff();
    for (int t = 0; t < QT; t += 8) {
      const uint4 u = *(const uint4*)&sm.kt[d][qq * QT + t];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        m = fmaxf(m, fmaxf(__uint_as_float(w[i] << 16), __uint_as_float(w[i] & 0xFFFF0000u)));
    }
    sm.part[qq][d] = m;
  }
  __syncthreads();
  if (tid < D)
    sm.top[tid] = fmaxf(fmaxf(sm.part[0][tid], sm.part[1][tid]), fmaxf(sm.part[2][tid], sm.part[3][tid]));
  __syncthreads();
  for (int job = tid; job < 4 * D; job += kWriterThreads) {
    const int d = job % D, qq = job / D;
    const float m = sm.top[d];
    float acc = 0.0f;
    for (int t = 0; t < QT; t += 8) {
      uint4* cell = (uint4*)&sm.kt[d][qq * QT + t];
      const uint4 u = *cell;
      uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float k0 = __uint_as_float(w[i] << 16);
        const float k1 = __uint_as_float(w[i] & 0xFFFF0000u);
        const float e0 = exp_bf(rbf(k0 - m));
        const float e1 = exp_bf(rbf(k1 - m));
        acc += e0;
        acc += e1;
        w[i] = (uint32_t)f2bf(e0) | ((uint32_t)f2bf(e1) << 16);
      }
      *cell = make_uint4(w[0], w[1], w[2], w[3]);
    }
    sm.part[qq][d] = acc;
  }
  __syncthreads();
  if (tid < D) {
    const float total = rbf((sm.part[0][tid] + sm.part[1][tid]) + (sm.part[2][tid] + sm.part[3][tid]));
    sm.total[tid] = total;
    const float z = rbf(sm.top[tid] + log_bf(total));
    p.fine_z[((size_t)bh * p.fine_cap + slot) * D + tid] = f2bf(z);
  }
  __syncthreads();
  for (int job = tid; job < 4 * D; job += kWriterThreads) {
    const int d = job % D, qq = job / D;
    const float total = sm.total[d];
    const float inv = __builtin_amdgcn_rcpf(total);
    for (int t = 0; t < QT; t += 8) {
      uint4* cell = (uint4*)&sm.kt[d][qq * QT + t];
      const uint4 u = *cell;
      uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p0 = div_bf(__uint_as_float(w[i] << 16), total, inv);
        const float p1 = div_bf(__uint_as_float(w[i] & 0xFFFF0000u), total, inv);
        w[i] = pack_bf16x2(p0, p1);
      }
      *cell = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  __syncthreads();

  // ---- C^T = V^T P on MFMA 32x32x16 (the bank stores C^T[e][d], d
  // contiguous): the (TILES x TILES) output tiles are spread over 8 waves.
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, lk = (lane >> 5) * 8;
  constexpr int TILES = D / 32;
  constexpr int PER_WAVE = (TILES * TILES + 7) / 8;
  bf16_t* cdst = p.bank + ((size_t)bh * p.fine_cap + slot) * D * D;
  floatx16 acc[PER_WAVE];
#pragma unroll
  for (int t = 0; t < PER_WAVE; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
  const int tile0 = wave * PER_WAVE;
  if (tile0 < TILES * TILES) {
    for (int k0 = 0; k0 < kBlock; k0 += 16) {
#pragma unroll
      for (int t = 0; t < PER_WAVE; ++t) {
        const int rt = (tile0 + t) / TILES, ct = (tile0 + t) % TILES;
        const bf16x8 a = *(const bf16x8*)&sm.vt[rt * 32 + li][k0 + lk];
        const bf16x8 bv = *(const bf16x8*)&sm.kt[ct * 32 + li][k0 + lk];
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bv, acc[t], 0, 0, 0);
      }
    }
    // D layout: lane holds column li (d), rows (e) 8*(i/4) + 4*(lane/32) + i%4.
#pragma unroll
    for (int t = 0; t < PER_WAVE; ++t) {
      const int rt = (tile0 + t) / TILES, ct = (tile0 + t) % TILES;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = rt * 32 + 8 * (i / 4) + 4 * (lane >> 5) + (i % 4);
        cdst[(size_t)row * D + ct * 32 + li] = f2bf(acc[t][i]);
      }
    }
  }
}

template <int D>
__global__ __launch_bounds__(kThreads) void epilogue_kernel(EpilogueParams p) {
  __shared__ float pz_s[D];
  const int bh = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = p.slot / p.group;
  const int first = g * p.group;
  const int n = p.slot - first + 1;
  const bf16_t* z = p.fine_z + (size_t)bh * p.fine_cap * D;
  if (tid < D) {
    float zv[8];
    float m = -__builtin_inff();
    for (int i = 0; i < 8; ++i) {
      zv[i] = i < n ? bf2f(z[(size_t)(first + i) * D + tid]) : 0.0f;
      if (i < n) m = fmaxf(m, zv[i]);
    }
    if (__builtin_isinf(m)) m = 0.0f;
    float pz;
    if (p.recompute) {
      float e[8];
      for (int i = 0; i < 8; ++i) e[i] = i < n ? exp_bf(rbf(zv[i] - m)) : 0.0f;
      for (int w = 4; w >= 1; w >>= 1)
        for (int i = 0; i < w; ++i) e[i] += e[i + w];
      pz = rbf(log_bf(rbf(e[0])) + m);
    } else {
      pz = bf2f(p.page_z[((size_t)bh * p.page_cap + g) * D + tid]);
    }
    pz_s[tid] = pz;
    if (p.recompute) p.page_z[((size_t)bh * p.page_cap + g) * D + tid] = f2bf(pz);
    for (int i = 0; i < n; ++i)
      p.fine_sw[((size_t)bh * p.fine_cap + first + i) * D + tid] = f2bf(exp_bf(rbf(zv[i] - pz)));
  }
  __syncthreads();
  // page weights: one wave per channel, lanes over pages (butterfly order).
  const int P = p.pages;
  int width = 1;
  while (width * 64 < P) width <<= 1;
  const bf16_t* pzg = p.page_z + (size_t)bh * p.page_cap * D;
  bf16_t* pwg = p.page_w + (size_t)bh * p.page_cap * D;
  for (int d = wave; d < D; d += kThreads / 64) {
    float x[32];
    float m = -__builtin_inff();
    for (int k = 0; k < width; ++k) {
      const int pg = lane + 64 * k;
      x[k] = pg < P ? (pg == g ? pz_s[d] : bf2f(pzg[(size_t)pg * D + d])) : -__builtin_inff();
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
      if (pg < P) pwg[(size_t)pg * D + d] = f2bf(exp_cr(x[k] - m) / total);
    }
  }
}

}  // namespace

hipError_t launch_writer(const WriterParams& p, int head_dim, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  const dim3 grid((unsigned)(p.count * p.B * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(writer_kernel<128>, grid, dim3(kWriterThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(writer_kernel<64>, grid, dim3(kWriterThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_seal_epilogue(const EpilogueParams& p, int head_dim, hipStream_t s) {
  if (p.pages > 64 * 32) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(p.B * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(epilogue_kernel<128>, grid, dim3(kThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(epilogue_kernel<64>, grid, dim3(kThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace tao
