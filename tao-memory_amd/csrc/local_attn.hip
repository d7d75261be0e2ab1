// Exact local attention (suffix-aligned causal) on MFMA for gfx950.
//
// Restates flash_attn_func (flash_attention.py:16-37): softmax(QK^T/sqrt(D))V
// where query row i of a chunk sees keys up to its own absolute position and
// no key older than the chunk's window start. A plan tile (up to 256 queries
// of one (batch, head), one window start) runs as two workgroups of 4 waves,
// 128 queries each; wave w owns 32 queries. Two such workgroups share a CU
// (about 200 VGPRs a lane, 64 KB of LDS at D = 128), each with its own
// barriers, so one's softmax VALU runs while the other's MFMAs do.
//
// Keys stream in 64-key blocks through two LDS stages. Every K and V row is
// copied from global memory straight into LDS (global_load_lds_dwordx4: a
// wave's 64 lanes fill 1 KB of consecutive LDS), the next block's copies in
// flight while the current block computes; rows past the window's end copy
// the last existing row (their scores are masked). Rows keep their 16-byte
// chunks XOR-swizzled (K by row % 16, V by 2 * row % 16 at D = 128), so the
// operand reads below meet distinct banks.
//
// Per 64-key block and wave:
//   S^T[key, query] = K . Q^T      v_mfma_f32_32x32x16_bf16; K rows from LDS
//                                  (ds_read_b128), Q in VGPRs
//   online softmax per query       each lane owns one query column
//   O^T[d, query]  += V^T . P^T    P^T comes straight from the S^T
//                                  accumulators: the contraction runs over a
//                                  key permutation that matches the
//                                  accumulator layout (keys 4j .. 4j + 3 in
//                                  lane half j % 2), and V^T is read in that
//                                  order by ds_read_b64_tr_b16: within 16
//                                  lanes, lane i gets element i % 4 of the
//                                  8 bytes lane 4k + i / 4 addresses, k =
//                                  0..3, so lanes addressing a 4-key x
//                                  16-channel tile receive 4 consecutive keys
//                                  of their own channel.
// The row sums of P add the same bf16-rounded probabilities the P V
// product uses, two per v_dot2_f32_bf16.
// Keys older than kpos0 come from the token ring, newer ones from the call's
// key operands; query row r sits at absolute position qpos0 + r.
//
// The LDS stages are written by the copies themselves, which the compiler
// does not order against its own LDS reads; the kernel therefore reads them
// with explicit ds_read instructions and waits for them itself: each wave
// waits for its own copies (vmcnt) before the barrier that publishes a
// block, and for its reads (lgkmcnt) before using them.
#include "tao_launch.h"
#include "tao_common.h"
#include "tao_lds.h"

namespace tao {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kKeys = 64;                    // keys per block
constexpr int kLaWaves = 4;
constexpr int kLaThreads = 64 * kLaWaves;    // one 128-query half of a plan tile
constexpr int kHalfQ = 32 * kLaWaves;

template <int D>
struct LaGeo {
  static constexpr int CPR = D / 8;                   // 16-byte chunks per row
  static constexpr int TILE = kKeys * D * 2;          // bytes of one K or V block
  static constexpr int STAGE = 2 * TILE;              // K block, then V block
  static constexpr int LPW = TILE / 1024 / kLaWaves;  // 1 KB copies per wave and block
  static constexpr int KK = D / 16;                   // k-steps of S^T
  static constexpr int DT = D / 32;                   // 32-row tiles of O^T
};

constexpr int kRA = 4;   // K operand reads in flight ahead of their MFMA

TAO_DEV const bf16_t* key_row(const AttnParams& p, const TokView& tv, const bf16_t* ring,
                              int b, int h, long long pos, int D) {
  if (pos >= p.kpos0) return tv.p + b * tv.sb + (pos - p.kpos0) * tv.st + h * tv.sh;
  const int slot = (int)(pos % p.L);
  return ring + (((size_t)b * p.L + slot) * p.H + h) * D;
}

template <int D>
__global__ __launch_bounds__(kLaThreads, 2) void local_attn_kernel(AttnParams p) {
  using G = LaGeo<D>;
  constexpr int CPR = G::CPR, KK = G::KK, DT = G::DT, LPW = G::LPW;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * G::STAGE];
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int rest = blockIdx.x / BH;
  const int tile = rest >> 1, half = rest & 1;
  const int b = bh / p.H, h = bh % p.H;
  const int tcount = (int)min(p.tiles[3 * tile + 1], (int64_t)2 * kHalfQ);
  const long long first = p.tiles[3 * tile] + half * kHalfQ;
  const int count = min(tcount - half * kHalfQ, kHalfQ);
  if (count <= 0) return;                       // workgroup-uniform
  const long long key_start = p.tiles[3 * tile + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;

  const int nq = min(max(count - wave * 32, 0), 32);
  const bool qvalid = li < nq;
  // A wave past the half's last query (nq == 0) loads the half's first row.
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

  // ---- LDS addresses (stage 0; stage, sub-tile and row offsets are
  // immediates). K: row li of a 32-key sub-tile, chunk 2 kk + hl, swizzled
  // by row % CPR. V^T: lane s of 16-lane group g addresses key row
  // 4 (g / 2) + s / 4 (+ 8 for the second read, + 16 half, + 32 sub) and
  // channels t * 32 + 16 (g % 2) + 4 (s % 4) .. + 3, rows swizzled by
  // 2 * row % CPR.
  const uint32_t base = lds_addr(smem);
  uint32_t addr_k[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
    addr_k[kk] = base + (uint32_t)((li * CPR + ((2 * kk + hl) ^ (li & (CPR - 1)))) * 16);
  uint32_t addr_v[DT];
  {
    const int g = lane >> 4, s = lane & 15;
    const int row0 = 4 * (g >> 1) + (s >> 2);
    const int swz = (2 * row0) & (CPR - 1);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const int c = 4 * t + 2 * (g & 1) + ((s & 3) >> 1);
      addr_v[t] = base + (uint32_t)(G::TILE + (row0 * CPR + (c ^ swz)) * 16 + (s & 1) * 8);
    }
  }

  // ---- copies of one 64-key block into stage `st`. Copy i of this wave
  // fills 1 KB piece J = wave * LPW + i: lane L gets row (64 J + L) / CPR,
  // chunk position (64 J + L) % CPR, which holds the row's chunk
  // position ^ swizzle.
  // Rows at or after kpos0 come from the call's operands. When a whole block
  // does and the operands' row strides are small, each copy's address is the
  // block's (uniform) base plus a per-lane 32-bit byte offset fixed for the
  // kernel.
  const long long direct_from = p.kpos0;
  const bool small_strides = p.k.st >= 0 && p.v.st >= 0 && p.k.st < (1 << 22) &&
                             p.v.st < (1 << 22);
  uint32_t off_k[LPW], off_v[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int q = (wave * LPW + i) * 64 + lane, r = q / CPR, pos = q % CPR;
    off_k[i] = (uint32_t)(2 * (r * p.k.st + (pos ^ (r & (CPR - 1))) * 8));
    off_v[i] = (uint32_t)(2 * (r * p.v.st + (pos ^ ((2 * r) & (CPR - 1))) * 8));
  }
  auto issue = [&](long long kb, int st) __attribute__((always_inline)) {
    unsigned char* kdst = smem + st * G::STAGE;
    unsigned char* vdst = kdst + G::TILE;
    const bool fast = small_strides && kb >= direct_from && kb + kKeys <= kend;   // uniform
    if (fast) {
      const char* kb_base = (const char*)(p.k.p + b * p.k.sb + (kb - p.kpos0) * p.k.st + h * p.k.sh);
      const char* vb_base = (const char*)(p.v.p + b * p.v.sb + (kb - p.kpos0) * p.v.st + h * p.v.sh);
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int J = wave * LPW + i;
        __builtin_amdgcn_global_load_lds((const void*)(kb_base + off_k[i]),
                                         (lds_void_t*)(kdst + J * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(vb_base + off_v[i]),
                                         (lds_void_t*)(vdst + J * 1024), 16, 0, 0);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int J = wave * LPW + i;
      const int q = J * 64 + lane, r = q / CPR, pos = q % CPR;
      const long long kp = kb + r < kend ? kb + r : kend - 1;
      __builtin_amdgcn_global_load_lds(
          key_row(p, p.k, p.ring_k, b, h, kp, D) + (pos ^ (r & (CPR - 1))) * 8,
          (lds_void_t*)(kdst + J * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          key_row(p, p.v, p.ring_v, b, h, kp, D) + (pos ^ ((2 * r) & (CPR - 1))) * 8,
          (lds_void_t*)(vdst + J * 1024), 16, 0, 0);
    }
  };

  floatx16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[t][i] = 0.0f;
  float lsum = 0.0f;
  float m_run = -__builtin_inff();

  // One block from stage ST: wait for it, start the next block's copies,
  // then (waves with queries that see it) scores, softmax and P V.
  auto block = [&](long long kb, auto stage) __attribute__((always_inline)) {
    constexpr int ST = decltype(stage)::value;
    constexpr int KOFF = ST * G::STAGE;
    wait_vm0();               // this wave's copies of the block landed
    __syncthreads();          // all copies landed; the other stage is free
    if (kb + kKeys < kend) issue(kb + kKeys, ST ^ 1);
    if (nq == 0 || kb > wave_last) return;      // uniform per wave

    floatx16 s[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[sub][i] = 0.0f;
    {
      // The 2 KK steps (sub-tile, k-step) in order, K operands read kRA
      // steps ahead through a register ring.
      constexpr int NS = 2 * KK;
      u32x4 ka[kRA];
      auto kread = [&](auto n_c) __attribute__((always_inline)) {
        constexpr int N = decltype(n_c)::value;
        ka[N % kRA] = ds_read16<KOFF + (N / KK) * 32 * CPR * 16>(addr_k[N % KK]);
      };
      unroll<kRA>([&](auto n_c) __attribute__((always_inline)) { kread(n_c); });
      unroll<NS>([&](auto n_c) __attribute__((always_inline)) {
        constexpr int N = decltype(n_c)::value;
        constexpr int AHEAD = (NS - 1 - N) < (kRA - 1) ? (NS - 1 - N) : (kRA - 1);
        wait_lgkm<AHEAD>(ka[N % kRA]);
        const u32x4 a = ka[N % kRA];
        s[N / KK] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(make_uint4(a.x, a.y, a.z, a.w)),
                                                          qreg[N % KK], s[N / KK], 0, 0, 0);
        if constexpr (N + kRA < NS) kread(std::integral_constant<int, N + kRA>());
      });
    }
    // S^T layout: lane holds query li, keys 8*(i/4) + 4*hl + i%4 of each
    // sub-tile. Only blocks that reach past the wave's first query or the
    // end of the window need the mask (32-bit offsets from the block start).
    const bool masked = kb + kKeys - 1 > wave_first || kb + kKeys > kend;
    float bmax = -__builtin_inff();
    if (masked) {
      const int q_off = (int)(qpos - kb);          // keys at offset > q_off are in the future
      const int end_off = (int)(kend - kb);        // keys at offset >= end_off do not exist
      const int lim = (q_off + 1 < end_off ? q_off + 1 : end_off) - 4 * hl;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int off = sub * 32 + 8 * (i / 4) + (i % 4);
          const float v = off < lim ? s[sub][i] : -__builtin_inff();
          s[sub][i] = v;
          bmax = fmaxf(bmax, v);
        }
    } else {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 16; i += 2) bmax = fmaxf(bmax, fmaxf(s[sub][i], s[sub][i + 1]));
    }
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(bmax),
                                                       __float_as_uint(bmax), false, false);
      bmax = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * scale_log2;
    }
    // Raise the reference (and rescale O, l) only past the slack; a query
    // with no visible key yet keeps m = -inf and a shift of 0, so every exp
    // below sees -inf and returns 0.
    if (__any(bmax > m_run + kSlack)) {
      const float m_new = fmaxf(m_run, bmax);
      // No visible key yet on this lane (both -inf): O and l are still 0.
      const float alpha = m_new == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      lsum *= alpha;
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
    // P in bf16 for the MFMA; l sums the same rounded values, two per
    // v_dot2_f32_bf16 against (1, 1).
    bf16x8 pb[2][2];
    const bf16x2 ones2 = __builtin_bit_cast(bf16x2, 0x3F803F80u);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          w[j] = pack_bf16x2(s[sub][8 * hf + 2 * j], s[sub][8 * hf + 2 * j + 1]);
          lsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[j]), ones2, lsum,
                                                 false);
        }
        pb[sub][hf] = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
      }
    // O^T += V^T P^T over the block's four 16-key steps (sub, hf): the lane
    // half hl of step (sub, hf) holds keys 32 sub + 16 hf + 4 hl + {0..3, 8..11}.
    constexpr int VOFF = KOFF;        // addr_v already includes the K tile
    // Step n = 2 sub + hf reads 2 DT transposed pieces; the next step's
    // reads are issued before this step's MFMAs.
    u32x2 vr[2][2 * DT];
    auto vread = [&](auto n_c) __attribute__((always_inline)) {
      constexpr int N = decltype(n_c)::value;
      constexpr int ROW = 16 * N;                 // 32 sub + 16 hf
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        vr[N % 2][2 * t] = ds_read_tr8<VOFF + ROW * CPR * 16>(addr_v[t]);
        vr[N % 2][2 * t + 1] = ds_read_tr8<VOFF + (ROW + 8) * CPR * 16>(addr_v[t]);
      }
    };
    vread(std::integral_constant<int, 0>());
    unroll<4>([&](auto n_c) __attribute__((always_inline)) {
      constexpr int N = decltype(n_c)::value;
      if constexpr (N + 1 < 4) {
        vread(std::integral_constant<int, N + 1>());
        wait_lgkm<2 * DT>(vr[N % 2][2 * DT - 1]);
      } else {
        wait_lgkm<0>(vr[N % 2][2 * DT - 1]);
      }
#pragma unroll
      for (int t = 0; t < 2 * DT - 1; ++t) after_waits(vr[N % 2][t]);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const u32x2 lo = vr[N % 2][2 * t], hi = vr[N % 2][2 * t + 1];
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y)),
                                                       pb[N / 2][N % 2], o[t], 0, 0, 0);
      }
    });
  };

  issue(key_start, 0);
  long long kb = key_start;
  for (; kb + kKeys < kend; kb += 2 * kKeys) {
    block(kb, std::integral_constant<int, 0>());
    block(kb + kKeys, std::integral_constant<int, 1>());
  }
  if (kb < kend) block(kb, std::integral_constant<int, 0>());
  if (!qvalid) return;
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum), __float_as_uint(lsum),
                                                     false, false);
    lsum = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  const float l_run = lsum;
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
  const dim3 grid((unsigned)(2 * p.n_tiles * p.B * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(local_attn_kernel<128>, grid, dim3(kLaThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(local_attn_kernel<64>, grid, dim3(kLaThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace tao
