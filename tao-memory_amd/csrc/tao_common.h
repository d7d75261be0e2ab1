// Shared device helpers for the TaoMemory gfx950 kernels.
//
// Numeric contract (identical to the CPU oracle):
//  * bf16 is stored as raw uint16; float->bf16 is round-to-nearest-even.
//  * exp/log feeding bf16 state are "correctly rounded fp32, then RNE to
//    bf16": the fast fp32 result is used unless it lies within a few fp32
//    ulps of a bf16 rounding boundary, where the fp64 value decides.
//  * exp inside fp32 softmax internals is fp64 exp rounded to fp32.
//  * fp32 sums that feed routing use the 64-lane butterfly order
//    ("fold halves": pad to a power of two, add upper half onto lower half).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;

#define TAO_DEV __device__ __forceinline__

TAO_DEV float bf2f(bf16_t v) { return __uint_as_float(((uint32_t)v) << 16); }

// fp32 -> bf16, round to nearest even: one v_cvt_pk_bf16_f32 on gfx950. It
// equals the integer RNE (add 0x7FFF + lsb, truncate) for every non-NaN fp32
// input, denormals and infinities included (checked exhaustively on MI355X);
// a NaN stays a NaN.
TAO_DEV bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// Two fp32 -> packed bf16 pair (low = a), one instruction.
TAO_DEV uint32_t pack_bf16x2(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const b2 v = __builtin_convertvector((f2){a, b}, b2);
  return __builtin_bit_cast(uint32_t, v);
}

// Round an fp32 value to bf16 precision and return it as fp32.
TAO_DEV float rbf(float f) { return bf2f(f2bf(f)); }

// True when fp32 `y` is within `margin` ulps of a bf16 rounding boundary.
TAO_DEV bool near_bf16_midpoint(float y, int margin) {
  int low = (int)(__float_as_uint(y) & 0xFFFFu);
  int dist = low - 0x8000;
  return dist <= margin && dist >= -margin;
}

// bf16(correctly rounded fp32 exp(x)). The fast value is the hardware 2^t
// at t = r32(x * log2 e): for |x| <= 8 the argument's rounding and the
// rounded log2 e move it by under 8 fp32 ulps, plus the hardware exp's own
// ulp. Near a bf16 rounding boundary (16 ulps), or for |x| > 8, the fp64 exp
// decides. Every kernel call site passes a bf16 x, and all 65536 of them are
// checked against the correctly rounded reference.
// exp_fast / exp_needs_exact / exp_exact are the pieces, for callers that
// batch the (rare) fp64 fix-ups of several values behind one branch.
TAO_DEV float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269502f); }

TAO_DEV bool exp_needs_exact(float x, float y) {
  return near_bf16_midpoint(y, 16) || !(__builtin_fabsf(x) <= 8.0f);
}

TAO_DEV float exp_exact(float x) { return (float)exp((double)x); }

TAO_DEV float exp_bf(float x) {
  float y = exp_fast(x);
  if (exp_needs_exact(x, y)) y = exp_exact(x);
  return rbf(y);
}

// bf16(correctly rounded fp32 log(x)); zero, negative, denormal and
// non-finite inputs take the fp64 log.
TAO_DEV float log_bf(float x) {
  float y = logf(x);
  if (near_bf16_midpoint(y, 16) || !(x >= 1.17549435e-38f && x < __builtin_inff()))
    y = (float)log((double)x);
  return rbf(y);
}

// A feature-mass page descriptor (tao_stream.py:280-283, 483) of the n
// fines from `mass` (a page's first fine) at stride `stride`: r(log) of the
// fp32 mass total that fine_mass holds at the n-th of them (the run's sum in
// seal order through it).
TAO_DEV float mass_page_z(const float* mass, int n, size_t stride) {
  return log_bf(mass[(size_t)(n - 1) * stride]);
}

// Correctly rounded fp32 exp (fp64 evaluation).
TAO_DEV float exp_cr(float x) { return (float)exp((double)x); }

// Correctly rounded fp32 natural log (fp64 evaluation).
TAO_DEV float log_cr(float x) { return (float)log((double)x); }

// ---------------------------------------------------------------- wave ops
TAO_DEV float wave_sum_fold(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// The same fold without LDS round trips, on the bit-reversed layout: element
// e of a 64-element vector sits in lane fold_lane(e) = bitrev6(e) (an
// involution: lane L holds element fold_lane(L)). The fold's pairs
// (e, e ^ 32), (e, e ^ 16), ..., (e, e ^ 1) are then the lane pairs
// (L, L ^ 1), (L, L ^ 2), ..., (L, L ^ 32). Levels 1-2 are quad_perm DPP
// adds; afterwards a quad holds one value, so the half-row mirror
// (L -> 7 - L in 8 lanes) reaches the partner quad, and then the row mirror
// (L -> 15 - L) the partner 8-lane group; the last two levels add the four
// row totals of lanes 0, 16, 32, 48. fp32 addition is commutative, so every
// partial sum equals wave_sum_fold's on the natural layout bit for bit. The
// result is uniform across the wave.
TAO_DEV int fold_lane(int e) { return (int)(__builtin_bitreverse32((uint32_t)e) >> 26); }

template <int CTRL>
TAO_DEV float dpp_partner(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

TAO_DEV float wave_fold_sum(float v) {
  v += dpp_partner<0xB1>(v);     // quad_perm [1, 0, 3, 2]: lane ^ 1
  v += dpp_partner<0x4E>(v);     // quad_perm [2, 3, 0, 1]: lane ^ 2
  v += dpp_partner<0x141>(v);    // row_half_mirror: the other quad of 8 lanes
  v += dpp_partner<0x140>(v);    // row_mirror: the other 8 lanes of the row
  const int bits = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 48));
  return (r0 + r1) + (r2 + r3);
}

// wave_fold_sum of N independent values at once, level by level across the
// values so their DPP steps interleave (no hazard stalls between the steps
// of one chain). Each result equals wave_fold_sum of that value bit for bit.
template <int N>
TAO_DEV void wave_fold_sum_n(float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_partner<0xB1>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_partner<0x4E>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_partner<0x141>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_partner<0x140>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int bits = __builtin_bit_cast(int, v[i]);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 48));
    v[i] = (r0 + r1) + (r2 + r3);
  }
}

// Maximum over the wave with the same DPP pattern (order-free).
TAO_DEV float wave_fold_max(float v) {
  v = fmaxf(v, dpp_partner<0xB1>(v));
  v = fmaxf(v, dpp_partner<0x4E>(v));
  v = fmaxf(v, dpp_partner<0x141>(v));
  v = fmaxf(v, dpp_partner<0x140>(v));
  const int bits = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Device-coherent (agent-scope) relaxed accesses: once a store made this way
// has been acknowledged (the storing wave's `s_waitcnt vmcnt(0)`, which the
// caller issues explicitly: a relaxed atomic carries no wait of its own), an
// agent-scope load on any XCD returns it. The single-launch decode step
// publishes its per-workgroup records with them, so no L2 write-back fence is
// needed between its workgroups.
TAO_DEV void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
TAO_DEV float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// XCD-affine workgroup numbering. The dispatcher hands workgroup i to XCD
// i % 8 (round-robin over the eight XCDs); remapping i so that the `per`
// workgroups of unit u (a batch-row x head) all get u % 8 keeps a head's
// decode kernels, its route fold and its combine on one XCD, so the data one
// kernel writes for a head (records, the folded route) and the ring window
// it re-reads every step sit in that XCD's L2. Returns (u, j), j < per; a
// bijection of [0, units * per). Units not a multiple of 8: plain order.
TAO_DEV void xcd_unit(int i, int units, int per, int& u, int& j) {
  const bool plain = (units & 7) != 0;      // selects, not branches: one division
  const int n = plain ? i : i >> 3;
  const int q = n / per;
  j = n - q * per;
  u = plain ? q : (i & 7) + 8 * q;
}

TAO_DEV float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Monotone 32-bit key of a bf16 score: larger score -> larger key.
TAO_DEV uint32_t bf16_order_key(bf16_t b) {
  uint32_t u = b;
  return (u & 0x8000u) ? (~u & 0xFFFFu) : (u | 0x8000u);
}

// Local-window length before appending the token at `position`:
// p for p < serve_limit, else keep + (p - serve_limit) mod fine.
TAO_DEV int local_len_at(long long position, int keep, int fine) {
  long long limit = keep + fine;
  if (position < limit) return (int)position;
  return keep + (int)((position - limit) % fine);
}

// Sealed fine memories before the token at `position` (the window seals
// its oldest `fine` tokens each time it reaches keep + fine).
TAO_DEV long long fines_before(long long position, int keep, int fine) {
  const long long limit = keep + fine;
  return position < limit ? 0 : (position - limit) / fine + 1;
}

// Page weights of one channel on one wave: r(softmax over P <= 2048 page
// descriptors), lane + 64 k -> page, the exps correctly rounded and summed
// in the oracle's butterfly order (fold the k halves, then the lanes).
// desc(pg) returns descriptor pg, write(pg, w) stores its weight.
template <typename Desc, typename Write>
TAO_DEV void page_weights_wave(int lane, int P, Desc desc, Write write) {
  if (P <= 64) {   // one page per lane (contexts up to 128K tokens)
    const float x = lane < P ? desc(lane) : -__builtin_inff();
    const float m = wave_max(x);
    const float e = lane < P ? exp_cr(x - m) : 0.0f;
    const float total = wave_sum_fold(e);
    if (lane < P) write(lane, f2bf(e / total));
    return;
  }
  int width = 1;
  while (width * 64 < P) width <<= 1;
  float x[32];
  float m = -__builtin_inff();
  for (int k = 0; k < width; ++k) {
    const int pg = lane + 64 * k;
    x[k] = pg < P ? desc(pg) : -__builtin_inff();
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
    if (pg < P) write(pg, f2bf(exp_cr(x[k] - m) / total));
  }
}

// Page descriptor of n <= 8 fine descriptors of one channel: torch's bf16
// logsumexp composite r(r(log r(sum r(exp r(z - m)))) + m), butterfly sum,
// infinite maximum replaced by 0 (tao_stream.py:283, 412, 485).
TAO_DEV float group_logsumexp(const float z[8], int n) {
  float m = -__builtin_inff();
  for (int i = 0; i < n; ++i) m = fmaxf(m, z[i]);
  if (__builtin_isinf(m)) m = 0.0f;
  float e[8];
  for (int i = 0; i < 8; ++i) e[i] = i < n ? exp_bf(rbf(z[i] - m)) : 0.0f;
  for (int w = 4; w >= 1; w >>= 1)
    for (int i = 0; i < w; ++i) e[i] += e[i + w];
  return rbf(log_bf(rbf(e[0])) + m);
}

