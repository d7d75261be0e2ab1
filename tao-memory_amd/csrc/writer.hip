// Softmax fine writer and seal epilogue for gfx950.
//
// writer_kernel: one workgroup of D / 32 waves per (block, batch, head).
// Restates _seal's softmax branch (tao_stream.py:66-77) for a 256-token
// block:
//   per channel d: m = max_t k, e = r(exp(r(k - m))), Z = r(sum_t e),
//   P = r(e / Z), z = r(m + r(log Z)); C = r(P^T V) with fp32 accumulation.
// z feeds routing and is bit-exact: the token sum uses the oracle's order
// (four 64-token quarters summed sequentially, then (q0+q1)+(q2+q3)). C only
// feeds reads (bf16 tolerance), so the kernel contracts the rounded e and
// scales each column by 1/Z, C = r((sum_t e V) / Z), instead of rounding
// P = e / Z element by element, within a bf16 ulp of P's rounding.
//
// C^T = V^T E runs on v_mfma_f32_32x32x16_bf16 with E as the B operand:
// wave w owns key channels 32 w .. 32 w + 31, lane (i, hl) channel 32 w + i
// and, for k-step ks, tokens 8 ks + 128 hl .. + 7 (a token permutation both
// operands share), so lane half 0 holds tokens 0..127 and half 1 tokens
// 128..255, each in order. The block's raw keys are copied from global
// memory straight into LDS (global_load_lds_dwordx4; rows row-major, each
// row's 16-byte chunks XOR-swizzled by 2 * row % (D / 8) so the reads below
// meet distinct banks) and read into registers in that layout with
// ds_read_b64_tr_b16 (4 consecutive tokens of one channel per read). The
// values are then copied into the same 64 KB while the column softmax runs
// in registers:
//   m: the lane's 128 maxima, then its partner half's (a lane swap);
//   e = r(exp(r(k - m))): the hardware exp, fp64 exp near a bf16 rounding
//      boundary or for |x| > 8, one branch per 8 values;
//   the quarter sums in token order as e is formed (quarters 0, 1 in lane
//      half 0, quarters 2, 3 in half 1), then (q0+q1)+(q2+q3) by a swap.
// Each wave then forms its 32 columns of C^T for all D value rows (V^T by
// transposed reads), scales them by 1/Z and writes them into the bank slot
// as C^T[e][d] (the contraction index d contiguous for every reader): no
// repack.
//
// epilogue_kernel: one wave per (batch, head, channel) after sealing fine `slot`
// (append_fine, tao_stream.py:477-501, plus the pending summary :277-290
// and the seal-epoch memo :399-416): page descriptor
// pz = logsumexp over the slot's group (torch's bf16 composite), segment
// weights sw = r(exp(r(z - pz))) of the group's fines, and page weights
// pw = r(softmax over pages) for every current page.
#include "tao_launch.h"
#include "tao_common.h"
#include "tao_lds.h"

namespace tao {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBlock = 256;                 // tokens per fine block

template <int D>
struct WGeo {
  static constexpr int WAVES = D / 32;                 // one 32-channel column tile each
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int CPR = D / 8;                    // 16-byte chunks per row
  static constexpr int RB = D * 2;                     // bytes per row
  static constexpr int TILE = kBlock * RB;             // bytes of the K (or V) block
  static constexpr int CPW = TILE / 1024 / WAVES;      // 1 KB copies per wave and tile
  static constexpr int KS = kBlock / 16;               // k-steps
  static constexpr int RT = D / 32;                    // 32-row tiles of value channels
};

// Chunk c of row r sits at chunk position c ^ swz(r).
template <int D>
TAO_DEV int swz(int r) { return (2 * r) & (D / 8 - 1); }

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

TAO_DEV float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
TAO_DEV float hi_bf(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

template <int D>
__global__ __launch_bounds__(WGeo<D>::THREADS) void writer_kernel(WriterParams p) {
  using G = WGeo<D>;
  constexpr int CPR = G::CPR, RB = G::RB, CPW = G::CPW, KS = G::KS;
  __shared__ __attribute__((aligned(1024))) unsigned char buf[G::TILE];
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int blk = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const long long start = p.starts[blk];
  const int slot = p.first_slot + blk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hl = lane >> 5;
  const long long rel = start - p.new_base;
  const int slot0 = (int)(start % p.L);
  const uint32_t base = lds_addr(buf);

  // ---- copies of a K or V block into buf. Copy i of this wave fills 1 KB
  // piece J = wave * CPW + i: lane L gets row (64 J + L) / CPR at chunk
  // position (64 J + L) % CPR, which holds the row's chunk position ^ swz.
  const bool fast = rel >= 0 && p.rk.st >= 0 && p.v.st >= 0 && p.rk.st < (1 << 21) &&
                    p.v.st < (1 << 21);                          // workgroup-uniform
  auto copy = [&](const TokView& tv, const bf16_t* ring) __attribute__((always_inline)) {
    const char* src0 = (const char*)(tv.p + b * tv.sb + (fast ? rel : 0) * tv.st + h * tv.sh);
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int J = wave * CPW + i, q = J * 64 + lane, r = q / CPR, pos = q % CPR;
      const int chunk = pos ^ swz<D>(r);
      const void* src =
          fast ? (const void*)(src0 + (uint32_t)(2 * (r * tv.st + chunk * 8)))
               : (const void*)(block_row(p, tv, ring, b, h, rel, slot0, r, D) + chunk * 8);
      __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(buf + J * 1024), 16, 0, 0);
    }
  };

  // Transposed-read addresses: lane s of lane group g (gh = g % 2) reads
  // rows 8 ks + 128 hl + 4 r + s / 4 (r = 0, 1), channels
  // cbase + 16 gh + 4 (s % 4) .. + 3; k-steps are immediate offsets (8 ks
  // rows move no swizzle).
  const int s = lane & 15, gh = (lane >> 4) & 1;
  auto tr_addr = [&](int cbase, int r) __attribute__((always_inline)) {
    const int row = 128 * hl + 4 * r + (s >> 2);
    const int chunk = (cbase >> 3) + 2 * gh + ((s & 3) >> 1);
    return base + (uint32_t)(row * RB + ((chunk ^ swz<D>(row)) * 16) + (s & 1) * 8);
  };

  copy(p.rk, p.ring_raw);
  wait_vm0();
  __syncthreads();

  // ---- keys of channel 32 w + li, tokens of this lane half, as B operands
  const uint32_t ak0 = tr_addr(32 * wave, 0), ak1 = tr_addr(32 * wave, 1);
  u32x2 ev[KS][2];
  unroll<KS>([&](auto ks_c) __attribute__((always_inline)) {
    constexpr int K = decltype(ks_c)::value;
    ev[K][0] = ds_read_tr8<K * 8 * RB>(ak0);
    ev[K][1] = ds_read_tr8<K * 8 * RB>(ak1);
  });
  wait_lgkm<0>(ev[KS - 1][1]);
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    after_waits(ev[k][0]);
    if (k < KS - 1) after_waits(ev[k][1]);
  }
  __syncthreads();                         // every wave has its keys: buf is free
  if (!p.z_only) copy(p.v, p.ring_v);      // values land while the softmax runs

  // ---- column maximum over the 256 tokens (lane half, then the partner)
  float m = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < KS; ++k)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t w0 = ev[k][r].x, w1 = ev[k][r].y;
      m = fmaxf(m, __builtin_fmaxf(fmaxf(lo_bf(w0), hi_bf(w0)), fmaxf(lo_bf(w1), hi_bf(w1))));
    }
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false,
                                                     false);
    m = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
  }

  // ---- e = r(exp(r(k - m))) in place, and the quarter sums in token order.
  // Eight exps, then one (rarely taken) branch for their fp64 fix-ups: the
  // closest low half-word to the bf16 rounding boundary and the largest |x|
  // of the eight decide it (exp_needs_exact for all eight).
  float qs[2] = {0.0f, 0.0f};
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    const uint32_t w[4] = {ev[k][0].x, ev[k][0].y, ev[k][1].x, ev[k][1].y};
    float x[8], y[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = rbf(lo_bf(w[i]) - m);
      x[2 * i + 1] = rbf(hi_bf(w[i]) - m);
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
    uint32_t e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[i] = pack_bf16x2(y[2 * i], y[2 * i + 1]);
      qs[k / (KS / 2)] += lo_bf(e[i]);
      qs[k / (KS / 2)] += hi_bf(e[i]);
    }
    ev[k][0].x = e[0];
    ev[k][0].y = e[1];
    ev[k][1].x = e[2];
    ev[k][1].y = e[3];
  }
  float total;
  {
    // lane half 0: q0 + q1, half 1: q2 + q3; Z = r((q0 + q1) + (q2 + q3))
    // (the swap returns the lane's own value and its partner's; the
    // partner is whichever is not the own one, or either when they agree)
    const float half_sum = qs[0] + qs[1];
    const uint32_t own = __float_as_uint(half_sum);
    const auto sw = __builtin_amdgcn_permlane32_swap(own, own, false, false);
    const float partner = __uint_as_float(sw[0] == own ? sw[1] : sw[0]);
    total = hl == 0 ? rbf(half_sum + partner) : rbf(partner + half_sum);
  }
  if (hl == 0)
    p.fine_z[((size_t)bh * p.fine_cap + slot) * D + 32 * wave + li] = f2bf(rbf(m + log_bf(total)));
  if (p.z_only) return;                    // workgroup-uniform

  // ---- C^T[e][32 w + li] = sum_t V^T[e][t] E[t][32 w + li] / Z
  wait_vm0();                              // this wave's value copies landed
  __syncthreads();
  uint32_t av[G::RT][2];
#pragma unroll
  for (int rt = 0; rt < G::RT; ++rt) {
    av[rt][0] = tr_addr(32 * rt, 0);
    av[rt][1] = tr_addr(32 * rt, 1);
  }
  floatx16 acc[G::RT];
#pragma unroll
  for (int rt = 0; rt < G::RT; ++rt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[rt][i] = 0.0f;
  unroll<KS>([&](auto ks_c) __attribute__((always_inline)) {
    constexpr int K = decltype(ks_c)::value;
    u32x2 va[G::RT][2];
#pragma unroll
    for (int rt = 0; rt < G::RT; ++rt) {
      va[rt][0] = ds_read_tr8<K * 8 * RB>(av[rt][0]);
      va[rt][1] = ds_read_tr8<K * 8 * RB>(av[rt][1]);
    }
    wait_lgkm<0>(va[G::RT - 1][1]);
    const bf16x8 eb = as_bf16x8(make_uint4(ev[K][0].x, ev[K][0].y, ev[K][1].x, ev[K][1].y));
#pragma unroll
    for (int rt = 0; rt < G::RT; ++rt) {
      after_waits(va[rt][0]);
      if (rt < G::RT - 1) after_waits(va[rt][1]);
      acc[rt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          as_bf16x8(make_uint4(va[rt][0].x, va[rt][0].y, va[rt][1].x, va[rt][1].y)), eb, acc[rt],
          0, 0, 0);
    }
  });
  // D layout: lane holds column li (d), rows (e) 8*(i/4) + 4*hl + i%4.
  const float inv = __builtin_amdgcn_rcpf(total);
  bf16_t* cdst = p.bank + ((size_t)bh * p.fine_cap + slot) * D * D + 32 * wave + li;
#pragma unroll
  for (int rt = 0; rt < G::RT; ++rt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = rt * 32 + 8 * (i / 4) + 4 * hl + (i % 4);
      cdst[(size_t)row * D] = f2bf(acc[rt][i] * inv);
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
  const dim3 grid((unsigned)(p.count * p.B * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(writer_kernel<128>, grid, dim3(WGeo<128>::THREADS), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(writer_kernel<64>, grid, dim3(WGeo<64>::THREADS), 0, s, p);
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
