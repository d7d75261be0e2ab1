// Exact local attention (suffix-aligned causal) on MFMA for gfx950.
//
// Restates flash_attn_func (flash_attention.py:16-37): softmax(QK^T/sqrt(D))V
// where query row i of a chunk sees keys up to its own absolute position and
// no key older than the chunk's window start. One workgroup = one tile of up
// to 256 queries of one (batch, head); wave w owns 32 queries. The next
// 64-key block is fetched into registers while the current one computes.
//
// Per 64-key block (staged in LDS: K row-major, V transposed):
//   S^T[key, query] = K . Q^T         v_mfma_f32_32x32x16_bf16, Q in VGPRs
//   online softmax per query          each lane owns one query column
//   O^T[d, query]  += V^T . P^T       P^T comes straight from the S^T
//                                     accumulators: the contraction runs over
//                                     a key permutation that matches the
//                                     accumulator layout, and V^T is read
//                                     with the same permutation.
// Keys older than kpos0 come from the token ring, newer ones from the call's
// key operands; query row r sits at absolute position qpos0 + r.
#include "tao_launch.h"
#include "tao_common.h"

namespace tao {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kKeys = 64;
constexpr int kAttnThreads = 512;   // 8 waves x 32 queries = 256-query tiles

// V^T rows are padded to 68 keys (34 dwords): 16 lanes reading 8 bytes
// from 16 consecutive channel rows land on distinct banks, and the
// transposing 4-byte writes put a half-wave on one row's consecutive key
// pairs.
template <int D>
struct AttnSmem {
  bf16_t k[kKeys][D + 8];
  bf16_t vt[D][kKeys + 4];
};

TAO_DEV const bf16_t* key_row(const AttnParams& p, const TokView& tv, const bf16_t* ring,
                              int b, int h, long long pos, int D) {
  if (pos >= p.kpos0) return tv.p + b * tv.sb + (pos - p.kpos0) * tv.st + h * tv.sh;
  const int slot = (int)(pos % p.L);
  return ring + (((size_t)b * p.L + slot) * p.H + h) * D;
}

TAO_DEV bf16x8 as_bf16x8(const uint4& u) {
  bf16x8 r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

template <int D>
__global__ __launch_bounds__(kAttnThreads) void local_attn_kernel(AttnParams p) {
  __shared__ AttnSmem<D> sm;
  constexpr int CH = D / 8;
  constexpr int DT = D / 32;    // 32-row tiles of O^T
  constexpr int KK = D / 16;    // k-steps of S^T
  constexpr int KJ = (kKeys * CH + kAttnThreads - 1) / kAttnThreads;        // K row jobs
  constexpr int VJ = ((kKeys / 2) * CH + kAttnThreads - 1) / kAttnThreads;  // V pair jobs
  const int bh = blockIdx.x % (p.B * p.H);
  const int tile = blockIdx.x / (p.B * p.H);
  const int b = bh / p.H, h = bh % p.H;
  const long long first = p.tiles[3 * tile];
  const int count = (int)p.tiles[3 * tile + 1];
  const long long key_start = p.tiles[3 * tile + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;

  const int nq = min(max(count - wave * 32, 0), 32);
  const bool qvalid = li < nq;
  // A wave past the tile's last query (nq == 0) loads the tile's first row:
  // first + 32 * wave may lie beyond the operand.
  const long long qtok = first + (nq > 0 ? wave * 32 + min(li, nq - 1) : 0);
  const long long qpos = p.qpos0 + qtok;
  const long long wave_last = p.qpos0 + first + wave * 32 + nq - 1;
  const long long wave_first = p.qpos0 + first + wave * 32;
  const long long kend = p.qpos0 + first + count;   // exclusive

  bf16x8 qreg[KK];
  {
    const bf16_t* qrow = p.q.p + b * p.q.sb + qtok * p.q.st + h * p.q.sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qreg[kk] = as_bf16x8(*(const uint4*)(qrow + 16 * kk + 8 * hl));
  }
  const float scale_log2 = (float)(1.4426950408889634 / __builtin_sqrt((double)D));
  // Online softmax with a lazily raised reference: p = 2^(s * c - m) with
  // m (log2 units) raised only when a block's maximum exceeds it by more
  // than kSlack, so O and l are rescaled rarely; o / l is independent of the
  // reference and p <= 2^kSlack stays well inside bf16's range.
  constexpr float kSlack = 8.0f;

  // Global loads of one 64-key block into registers (prefetch). When the
  // whole window lies in the call's operands (no ring rows: training and
  // first prefills), each thread walks fixed row offsets with pointers that
  // advance 64 rows a block; otherwise every row goes through key_row.
  const bool direct = key_start >= p.kpos0;          // workgroup-uniform
  uint4 kpre[KJ], va[VJ], vb[VJ];
  const bf16_t* kptr[KJ];
  const bf16_t* vptr[VJ];
  const int64_t step_k = (int64_t)kKeys * p.k.st, step_v = (int64_t)kKeys * p.v.st;
  if (direct) {
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int job = min(tid + j * kAttnThreads, kKeys * CH - 1);
      kptr[j] = p.k.p + b * p.k.sb + (key_start - p.kpos0 + job / CH) * p.k.st + h * p.k.sh +
                (job % CH) * 8;
    }
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
      const int job = min(tid + j * kAttnThreads, (kKeys / 2) * CH - 1);
      const int t0 = 2 * (job % (kKeys / 2)), c = job / (kKeys / 2);
      vptr[j] = p.v.p + b * p.v.sb + (key_start - p.kpos0 + t0) * p.v.st + h * p.v.sh + c * 8;
    }
  }
  auto fetch = [&](long long kb) {
    if (direct) {
      const int rem = (int)(kend - kb);              // rows of this block that exist
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int job = tid + j * kAttnThreads;
        kpre[j] = make_uint4(0, 0, 0, 0);
        if (job < kKeys * CH && job / CH < rem) kpre[j] = *(const uint4*)kptr[j];
        kptr[j] += step_k;
      }
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        const int job = tid + j * kAttnThreads;
        va[j] = make_uint4(0, 0, 0, 0);
        vb[j] = make_uint4(0, 0, 0, 0);
        if (job < (kKeys / 2) * CH) {
          const int t0 = 2 * (job % (kKeys / 2));
          if (t0 < rem) va[j] = *(const uint4*)vptr[j];
          if (t0 + 1 < rem) vb[j] = *(const uint4*)(vptr[j] + p.v.st);
        }
        vptr[j] += step_v;
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int job = tid + j * kAttnThreads;
      kpre[j] = make_uint4(0, 0, 0, 0);
      if (job < kKeys * CH && kb + job / CH < kend)
        kpre[j] = *(const uint4*)(key_row(p, p.k, p.ring_k, b, h, kb + job / CH, D) + (job % CH) * 8);
    }
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
      // job -> (channel chunk c, key pair): 32 consecutive jobs share c.
      const int job = tid + j * kAttnThreads;
      va[j] = make_uint4(0, 0, 0, 0);
      vb[j] = make_uint4(0, 0, 0, 0);
      if (job < (kKeys / 2) * CH) {
        const int t0 = 2 * (job % (kKeys / 2)), c = job / (kKeys / 2);
        if (kb + t0 < kend) va[j] = *(const uint4*)(key_row(p, p.v, p.ring_v, b, h, kb + t0, D) + c * 8);
        if (kb + t0 + 1 < kend) vb[j] = *(const uint4*)(key_row(p, p.v, p.ring_v, b, h, kb + t0 + 1, D) + c * 8);
      }
    }
  };

  floatx16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[t][i] = 0.0f;
  // Row sums of P on the matrix pipe: an A operand of ones gives
  // sum_k P[query][k] in every row of the accumulator (element 0 is used).
  floatx16 lacc;
#pragma unroll
  for (int i = 0; i < 16; ++i) lacc[i] = 0.0f;
  const bf16x8 ones = as_bf16x8(make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u));
  float m_run = -__builtin_inff();

  fetch(key_start);
  for (long long kb = key_start; kb < kend; kb += kKeys) {
    __syncthreads();          // previous block fully consumed
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int job = tid + j * kAttnThreads;
      if (job < kKeys * CH) *(uint4*)&sm.k[job / CH][(job % CH) * 8] = kpre[j];
    }
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
      const int job = tid + j * kAttnThreads;
      if (job < (kKeys / 2) * CH) {
        const int t0 = 2 * (job % (kKeys / 2)), c = job / (kKeys / 2);
        const uint32_t wa[4] = {va[j].x, va[j].y, va[j].z, va[j].w};
        const uint32_t wb[4] = {vb[j].x, vb[j].y, vb[j].z, vb[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          *(uint32_t*)&sm.vt[c * 8 + 2 * i][t0] = (wa[i] & 0xFFFFu) | (wb[i] << 16);
          *(uint32_t*)&sm.vt[c * 8 + 2 * i + 1][t0] = (wa[i] >> 16) | (wb[i] & 0xFFFF0000u);
        }
      }
    }
    __syncthreads();
    if (kb + kKeys < kend) fetch(kb + kKeys);   // overlaps the math below
    if (nq == 0 || kb > wave_last) continue;    // uniform per wave

    floatx16 s[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[sub][i] = 0.0f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const bf16x8 a = as_bf16x8(*(const uint4*)&sm.k[sub * 32 + li][16 * kk + 8 * hl]);
        s[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[kk], s[sub], 0, 0, 0);
      }
    }
    // S^T layout: lane holds query li, keys 8*(i/4) + 4*hl + i%4 of each
    // sub-tile. Only blocks that reach past the wave's first query or the
    // end of the window need the mask (32-bit offsets from the block start).
    const bool masked = kb + kKeys - 1 > wave_first || kb + kKeys > kend;
    float bmax = -__builtin_inff();
    if (masked) {
      const int q_off = (int)(qpos - kb);          // keys at offset > q_off are in the future
      const int end_off = (int)(kend - kb);        // keys at offset >= end_off do not exist
      const int lim = q_off + 1 < end_off ? q_off + 1 : end_off;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int off = sub * 32 + 8 * (i / 4) + 4 * hl + (i % 4);
          const float v = off < lim ? s[sub][i] : -__builtin_inff();
          s[sub][i] = v;
          bmax = fmaxf(bmax, v);
        }
    } else {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 16; ++i) bmax = fmaxf(bmax, s[sub][i]);
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64)) * scale_log2;
    // Raise the reference (and rescale O, l) only past the slack; a query
    // with no visible key yet keeps m = -inf and a shift of 0, so every exp
    // below sees -inf and returns 0.
    if (__any(bmax > m_run + kSlack)) {
      const float m_new = fmaxf(m_run, bmax);
      // No visible key yet on this lane (both -inf): O and l are still 0.
      const float alpha = m_new == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
      for (int i = 0; i < 16; ++i) lacc[i] *= alpha;
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[t][i] *= alpha;
      m_run = m_new;
    }
    const float m_use = m_run == -__builtin_inff() ? 0.0f : m_run;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        s[sub][i] = __builtin_amdgcn_exp2f(fmaf(s[sub][i], scale_log2, -m_use));

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
          const uint2 lo = *(const uint2*)&sm.vt[t * 32 + li][kbase];
          const uint2 hi = *(const uint2*)&sm.vt[t * 32 + li][kbase + 8];
          const uint4 u = make_uint4(lo.x, lo.y, hi.x, hi.y);
          o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(u), pb, o[t], 0, 0, 0);
        }
        lacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ones, pb, lacc, 0, 0, 0);
      }
  }
  if (!qvalid) return;
  const float l_run = lacc[0];
  if (p.lse && hl == 0) p.lse[((size_t)b * p.T + qtok) * p.H + h] = m_run + __log2f(l_run);
  const float inv = 1.0f / l_run;
  bf16_t* orow = p.out + (((size_t)b * p.T + qtok) * p.H + h) * D;
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const int d = t * 32 + 8 * (i / 4) + 4 * hl;
      uint2 packed;
      packed.x = (uint32_t)f2bf(o[t][i] * inv) | ((uint32_t)f2bf(o[t][i + 1] * inv) << 16);
      packed.y = (uint32_t)f2bf(o[t][i + 2] * inv) | ((uint32_t)f2bf(o[t][i + 3] * inv) << 16);
      *(uint2*)(orow + d) = packed;
    }
}

}  // namespace

hipError_t launch_local_attention(const AttnParams& p, int head_dim, hipStream_t s) {
  if (p.n_tiles <= 0) return hipSuccess;
  const dim3 grid((unsigned)(p.n_tiles * p.B * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(local_attn_kernel<128>, grid, dim3(kAttnThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(local_attn_kernel<64>, grid, dim3(kAttnThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace tao
