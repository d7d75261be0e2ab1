// Softmax fine writer and seal epilogue for gfx950.
//
// writer_kernel: one workgroup per (block, batch, head). Restates _seal's
// softmax branch (tao_stream.py:66-77) for a 256-token block:
//   per channel d: m = max_t k, e = r(exp(r(k - m))), Z = r(sum_t e),
//   P = r(e / Z), z = r(m + r(log Z)); C = r(P^T V) with fp32 accumulation.
// z feeds routing and is bit-exact: the token sum uses the oracle's order
// (four 64-token quarters summed sequentially, then (q0+q1)+(q2+q3)). C only
// feeds reads (bf16 tolerance), so the kernel contracts the rounded e and
// scales each column by 1/Z, C = r((sum_t e V) / Z), instead of rounding
// P = e / Z element by element: one VALU pass fewer per block, within a
// bf16 ulp of P's rounding.
// Two workgroups per block and head, one per half of the key channels d
// (the softmax is per channel): raw_k of the half and V are staged
// transposed in LDS ([channel][token], token contiguous; V in 64-token
// chunks) so both MFMA operands are 16-byte LDS reads; C^T = V^T E runs on
// v_mfma_f32_32x32x16_bf16. The bank keeps C^T[e][d] so the contraction
// index d is contiguous for every reader. C goes straight into its bank
// slot: no repack.
//
// epilogue_kernel: one wave per (batch, head, channel) after sealing fine `slot`
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
constexpr int kRowPad = kBlock + 8;         // K^T row stride in bf16 (528 B)
constexpr int kVChunk = 64;                 // tokens per staged V^T chunk
constexpr int kVPad = kVChunk + 4;          // V^T row stride in bf16 (34 dwords)
constexpr int kWriterThreads = 256;         // 4 waves

// One workgroup owns half of the key channels of one (block, batch, head):
// DH = D / 2 channels of K^T (then E^T) for all 256 tokens, and V^T of all
// D value channels streamed through one 64-token chunk. About 53 KB of LDS
// at D = 128, so three workgroups share a CU and one's exp pass overlaps the
// others' loads and MFMAs.
template <int D>
struct WriterSmem {
  bf16_t kt[D / 2][kRowPad];   // raw keys of the half, then e = r(exp(r(k - m)))
  bf16_t vt[D][kVPad];         // values of one token chunk, transposed
  float part[4][D / 2];
  float top[D / 2];
  float inv_z[D / 2];          // 1 / Z per channel of the half
};

// Row of token `t` of a block: token rel + t of the call's operands when
// rel + t >= 0 (rel = start - new_base), else ring slot (slot0 + t) mod L
// (slot0 = start mod L, t < 256 < L: at most one wrap).
TAO_DEV const bf16_t* block_row(const WriterParams& p, const TokView& tv, const bf16_t* ring,
                                int b, int h, long long rel, int slot0, int t, int D) {
  const long long r = rel + t;
  if (r >= 0) return tv.p + b * tv.sb + r * tv.st + h * tv.sh;
  int slot = slot0 + t;
  slot = slot >= p.L ? slot - p.L : slot;
  return ring + (((size_t)b * p.L + slot) * p.H + h) * D;
}

// Transposing LDS write of a token pair's 8 channels (16 bytes each):
// rows ch0 .. ch0 + 7 of dst receive the pair as one 4-byte word at column t0.
template <int STRIDE>
TAO_DEV void store_pair_t(bf16_t* dst, int ch0, int t0, const uint4& a, const uint4& b) {
  const uint32_t wa[4] = {a.x, a.y, a.z, a.w};
  const uint32_t wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    *(uint32_t*)&dst[(ch0 + 2 * i) * STRIDE + t0] = (wa[i] & 0xFFFFu) | (wb[i] << 16);
    *(uint32_t*)&dst[(ch0 + 2 * i + 1) * STRIDE + t0] = (wa[i] >> 16) | (wb[i] & 0xFFFF0000u);
  }
}

template <int D>
__global__ __launch_bounds__(kWriterThreads) void writer_kernel(WriterParams p) {
  constexpr int DH = D / 2;                     // channels of this workgroup
  constexpr int KJ = (kBlock / 2) * (DH / 8) / kWriterThreads;   // K token pairs per thread
  constexpr int VJ = (kVChunk / 2) * (D / 8) / kWriterThreads;   // V token pairs per thread
  constexpr int RT = D / 32, CT = DH / 32;      // 32 x 32 tiles of this half's C^T
  static_assert(KJ >= 1 && VJ >= 1, "head width 64 or 128");
  __shared__ WriterSmem<D> sm;
  const int BH = p.B * p.H;
  const int half = blockIdx.x % 2;
  const int bh = (blockIdx.x / 2) % BH;
  const int blk = blockIdx.x / (2 * BH);
  const int b = bh / p.H, h = bh % p.H;
  const long long start = p.starts[blk];
  const int slot = p.first_slot + blk;
  const int tid = threadIdx.x;
  const int d0 = half * DH;
  const long long rel = start - p.new_base;
  const int slot0 = (int)(start % p.L);

  // ---- issue the K half (all 256 tokens) and V chunk 0 loads. Job ->
  // (channel chunk c, token pair): 128 consecutive K jobs / 32 consecutive V
  // jobs share c, so the transposing writes fill consecutive words of a row.
  uint4 ka[KJ], kb[KJ], va[VJ], vb[VJ];
#pragma unroll
  for (int j = 0; j < KJ; ++j) {
    const int job = tid + j * kWriterThreads;
    const int c = job / (kBlock / 2), t0 = 2 * (job % (kBlock / 2));
    ka[j] = *(const uint4*)(block_row(p, p.rk, p.ring_raw, b, h, rel, slot0, t0, D) + d0 + c * 8);
    kb[j] = *(const uint4*)(block_row(p, p.rk, p.ring_raw, b, h, rel, slot0, t0 + 1, D) + d0 + c * 8);
  }
  auto load_v = [&](int chunk) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
      const int job = tid + j * kWriterThreads;
      const int c = job / (kVChunk / 2), t0 = chunk * kVChunk + 2 * (job % (kVChunk / 2));
      va[j] = *(const uint4*)(block_row(p, p.v, p.ring_v, b, h, rel, slot0, t0, D) + c * 8);
      vb[j] = *(const uint4*)(block_row(p, p.v, p.ring_v, b, h, rel, slot0, t0 + 1, D) + c * 8);
    }
  };
  load_v(0);
#pragma unroll
  for (int j = 0; j < KJ; ++j) {
    const int job = tid + j * kWriterThreads;
    store_pair_t<kRowPad>(&sm.kt[0][0], (job / (kBlock / 2)) * 8, 2 * (job % (kBlock / 2)),
                          ka[j], kb[j]);
  }
  __syncthreads();

  // ---- column softmax: jobs (channel d of the half, quarter of 64 tokens)
  constexpr int QT = kBlock / 4;
  for (int job = tid; job < 4 * DH; job += kWriterThreads) {
    const int d = job % DH, qq = job / DH;
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
  if (tid < DH)
    sm.top[tid] = fmaxf(fmaxf(sm.part[0][tid], sm.part[1][tid]), fmaxf(sm.part[2][tid], sm.part[3][tid]));
  __syncthreads();
  for (int job = tid; job < 4 * DH; job += kWriterThreads) {
    const int d = job % DH, qq = job / DH;
    const float m = sm.top[d];
    float acc = 0.0f;
    for (int t = 0; t < QT; t += 8) {
      uint4* cell = (uint4*)&sm.kt[d][qq * QT + t];
      const uint4 u = *cell;
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
      // Eight exps, then one (rarely taken) branch for their fp64 fix-ups:
      // the closest low half-word to the bf16 rounding boundary and the
      // largest |x| of the eight decide it (exp_needs_exact for all eight).
      float x[8], y[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[2 * i] = rbf(__uint_as_float(w[i] << 16) - m);
        x[2 * i + 1] = rbf(__uint_as_float(w[i] & 0xFFFF0000u) - m);
      }
      uint32_t near = 0xFFFFFFFFu;
      float big = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        y[i] = exp_fast(x[i]);
        near = min(near, (__float_as_uint(y[i]) & 0xFFFFu) - 0x7FF0u);
        big = fmaxf(big, __builtin_fabsf(x[i]));
      }
      if (near < 33u || !(big <= 8.0f)) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (exp_needs_exact(x[i], y[i])) y[i] = exp_exact(x[i]);
      }
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e0 = rbf(y[2 * i]), e1 = rbf(y[2 * i + 1]);
        acc += e0;
        acc += e1;
        o[i] = pack_bf16x2(e0, e1);
      }
      *cell = make_uint4(o[0], o[1], o[2], o[3]);
    }
    sm.part[qq][d] = acc;
  }
  __syncthreads();
  if (tid < DH) {
    const float total = rbf((sm.part[0][tid] + sm.part[1][tid]) + (sm.part[2][tid] + sm.part[3][tid]));
    sm.inv_z[tid] = __builtin_amdgcn_rcpf(total);
    const float z = rbf(sm.top[tid] + log_bf(total));
    p.fine_z[((size_t)bh * p.fine_cap + slot) * D + d0 + tid] = f2bf(z);
  }
  if (p.z_only) return;                         // workgroup-uniform

  // ---- C^T[e][d] = sum_t V^T[e][t] E[t][d] / Z[d] on MFMA 32x32x16: wave w
  // owns row tile w (value channels 32w ..) and the half's CT column tiles;
  // V^T arrives in 64-token chunks, the next chunk's loads in flight.
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, lk = (lane >> 5) * 8;
  floatx16 acc[CT];
#pragma unroll
  for (int t = 0; t < CT; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
#pragma unroll
  for (int chunk = 0; chunk < kBlock / kVChunk; ++chunk) {
    __syncthreads();   // e complete (chunk 0) / previous chunk consumed
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
      const int job = tid + j * kWriterThreads;
      store_pair_t<kVPad>(&sm.vt[0][0], (job / (kVChunk / 2)) * 8, 2 * (job % (kVChunk / 2)),
                          va[j], vb[j]);
    }
    __syncthreads();
    if (chunk + 1 < kBlock / kVChunk) load_v(chunk + 1);
    if (wave < RT) {
#pragma unroll
      for (int kk = 0; kk < kVChunk; kk += 16) {
        const bf16x8 a = *(const bf16x8*)&sm.vt[wave * 32 + li][kk + lk];
#pragma unroll
        for (int t = 0; t < CT; ++t) {
          const bf16x8 bv = *(const bf16x8*)&sm.kt[t * 32 + li][chunk * kVChunk + kk + lk];
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bv, acc[t], 0, 0, 0);
        }
      }
    }
  }
  if (wave >= RT) return;
  // D layout: lane holds column li (d), rows (e) 8*(i/4) + 4*(lane/32) + i%4.
  bf16_t* cdst = p.bank + ((size_t)bh * p.fine_cap + slot) * D * D;
#pragma unroll
  for (int t = 0; t < CT; ++t) {
    const float inv_z = sm.inv_z[t * 32 + li];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = wave * 32 + 8 * (i / 4) + 4 * (lane >> 5) + (i % 4);
      cdst[(size_t)row * D + d0 + t * 32 + li] = f2bf(acc[t][i] * inv_z);
    }
  }
}

// One wave per (batch, head, channel d); four channels per workgroup.
template <int D>
__global__ __launch_bounds__(kThreads) void epilogue_kernel(EpilogueParams p) {
  constexpr int CPB = kThreads / 64;
  const int bh = blockIdx.x / (D / CPB);
  const int lane = threadIdx.x & 63;
  const int d = (blockIdx.x % (D / CPB)) * CPB + (threadIdx.x >> 6);
  const int g = p.slot / p.group;
  const int first = g * p.group;
  const int n = p.slot - first + 1;
  const bf16_t* z = p.fine_z + (size_t)bh * p.fine_cap * D;
  float pz = 0.0f;
  if (lane == 0) {
    float zv[8];
    float m = -__builtin_inff();
    for (int i = 0; i < 8; ++i) {
      zv[i] = i < n ? bf2f(z[(size_t)(first + i) * D + d]) : 0.0f;
      if (i < n) m = fmaxf(m, zv[i]);
    }
    if (__builtin_isinf(m)) m = 0.0f;
    if (p.recompute && p.fine_mass) {
      pz = mass_page_z(p.fine_mass + ((size_t)bh * p.fine_cap + first) * D + d, n, D);
      p.page_z[((size_t)bh * p.page_cap + g) * D + d] = f2bf(pz);
    } else if (p.recompute) {
      float e[8];
      for (int i = 0; i < 8; ++i) e[i] = i < n ? exp_bf(rbf(zv[i] - m)) : 0.0f;
      for (int w = 4; w >= 1; w >>= 1)
        for (int i = 0; i < w; ++i) e[i] += e[i + w];
      pz = rbf(log_bf(rbf(e[0])) + m);
      p.page_z[((size_t)bh * p.page_cap + g) * D + d] = f2bf(pz);
    } else {
      pz = bf2f(p.page_z[((size_t)bh * p.page_cap + g) * D + d]);
    }
    for (int i = 0; i < n; ++i)
      p.fine_sw[((size_t)bh * p.fine_cap + first + i) * D + d] = f2bf(exp_bf(rbf(zv[i] - pz)));
  }
  pz = __shfl(pz, 0, 64);
  // Page weights of every current page for channel d.
  const bf16_t* pzg = p.page_z + (size_t)bh * p.page_cap * D;
  bf16_t* pwg = p.page_w + (size_t)bh * p.page_cap * D;
  page_weights_wave(
      lane, p.pages,
      [&](int pg) { return pg == g ? pz : bf2f(pzg[(size_t)pg * D + d]); },
      [&](int pg, bf16_t w) { pwg[(size_t)pg * D + d] = w; });
}

}  // namespace

hipError_t launch_writer(const WriterParams& p, int head_dim, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  const dim3 grid((unsigned)(2 * p.count * p.B * p.H));
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
  const dim3 grid((unsigned)(p.B * p.H * (head_dim / (kThreads / 64))));
  if (head_dim == 128)
    hipLaunchKernelGGL(epilogue_kernel<128>, grid, dim3(kThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(epilogue_kernel<64>, grid, dim3(kThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace tao
