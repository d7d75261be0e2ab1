// Fused single-token decode step for gfx950, and the route fold it reads.
//
// One launch per new token (replaces, per request x layer, the reference's
// q1 page-memo region tao_stream.py:418-433 + query_fresh_fine.py:8-75, the
// local SDPA flash_attention.py:25-29 over torch.cat'ed K/V
// tao_stream.py:927-930, and the fusion kernels fusion_pointwise.py:10-117):
//
// decode_step_kernel: per (batch, head) local_units(D) local-attention
//   workgroups and fine_units(D) fine-read workgroups.
//   local workgroup j takes keys [j*K, (j+1)*K) (K = local_keys(D)) of the
//   exact window (K and V rows from the ring, or the new token), scores
//   them (row sums on DPP lane moves), weights each thread's keys against
//   their maximum and merges the rows into a record (m, l, o[D]) with m in
//   log2 units; workgroup 0 also appends the new token to the ring. Its only
//   scalar input is the cursor (a kernel argument in eager launches,
//   header[0] in graphs).
//   fine-read workgroup f reads 32 rows of the folded route:
//   num[e] = h . G^T[e], and den = r(h . g) (h = r(softmax_D(raw_q)));
//   with the coarse value branch on, fine_units(D) more workgroups read 32
//   rows each of the folded coarse matrix the same way (coarse.hip).
//   Every workgroup publishes its record with device-coherent stores and
//   counts itself in on its head's arrival counter; the head's last
//   workgroup merges the local records in a fixed order,
//   fine = r(r(num) / den), coarse = r(h . Gc^T[e]), applies the fusion
//   epilogue for all D channels; the last head advances header[0] (the
//   cursor graph replays read).
//
// fold_kernel (per route refresh and per seal, not per token): the q1 read
// is linear in ch_m = h * w_m with w_m = pw[page(m)] * sw[m] independent of
// the query, so the selected fine memories fold into one D x D matrix per
// head: G^T[e][d] = sum_m w_m[d] C^T_m[e][d], g[d] = sum_m w_m[d]. A decode
// step then reads 64 KB of G per head instead of M matrices of 32 KB. The
// reference rounds ch twice to bf16 before its fp32 sums
// (query_fresh_fine.py:38-40, 47-48, 67); the fold keeps w and the sums in
// fp32, which moves the fine read by well under one bf16 ulp of its inputs.
//
// The records cross the eight XCD L2 caches as agent-scope stores and loads
// (coherent without an L2 write-back); a device-scope release fence per
// workgroup would cost more than a second launch on this part.
#include <type_traits>

#include <algorithm>

#include "tao_launch.h"
#include "tao_common.h"
#include "tao_fusion.h"

namespace tao {
namespace {

template <int D>
struct Geo {
  static constexpr int CH = D / 8;                 // 16-byte chunks per row
  static constexpr int ROWS = kThreads / CH;       // rows per load pass
  static constexpr int KEYS = local_keys(D);       // keys per local workgroup
  static constexpr int KPT = KEYS / ROWS;          // key rows per thread
  static constexpr int NLOC = local_units(D);
  static constexpr int NFINE = fine_units(D);
};
static_assert(kThreads == 256, "thread layouts below assume 256 threads");

constexpr int kWaves = kThreads / 64;

template <int D>
struct StepSmem {
  float wo[kWaves][D];            // each wave's weighted value sums
  float wm[kWaves], wl[kWaves];   // each wave's maximum and weight sum
};

TAO_DEV void unpack8(const uint4& u, float out[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

// Sum over the CH (8 or 16) consecutive lanes that share one key row, on
// DPP lane moves (no LDS round trips): the two quad swaps give quad sums, the
// half-row mirror adds the other quad of 8 lanes, the row mirror the other
// 8 lanes of 16. Every lane of the row ends with the row's sum.
template <int CH>
TAO_DEV float row_sum(float v) {
  static_assert(CH == 8 || CH == 16, "a key row spans 8 or 16 lanes");
  v += dpp_partner<0xB1>(v);
  v += dpp_partner<0x4E>(v);
  v += dpp_partner<0x141>(v);
  if constexpr (CH == 16) v += dpp_partner<0x140>(v);
  return v;
}

// Sum (max) over the rows of key data one wave holds: CH lanes per row,
// 64 / CH rows. Row pairs combine on lane swaps (row_ror:8 inside a 16-lane
// row for CH = 8, then v_permlane16_swap and v_permlane32_swap), in the
// fixed order ((r0 + r1) + (r2 + r3)) ...; every lane ends with the total.
template <int CH>
TAO_DEV float wave_rows_sum(float v) {
  static_assert(CH == 8 || CH == 16, "a key row spans 8 or 16 lanes");
  if constexpr (CH == 8) v += dpp_partner<0x128>(v);
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int CH>
TAO_DEV float wave_rows_max(float v) {
  static_assert(CH == 8 || CH == 16, "a key row spans 8 or 16 lanes");
  if constexpr (CH == 8) v = fmaxf(v, dpp_partner<0x128>(v));
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// One (request, head)'s operands of one decode step, shared by the
// single-request kernels (DecodeParams) and the batched ones (BatchStepParams).
struct StepReq {
  const bf16_t* q; const bf16_t* k; const bf16_t* v; const bf16_t* rq; const bf16_t* rk;
  bf16_t* ring_k; bf16_t* ring_v; bf16_t* ring_raw;   // slot 0 of this (state row, head)
  const float* fold_g; const float* fold_den; const float* coarse_g;   // this head's
  float* recs;                                        // this (request, head)'s records
  int n_old, first_slot;   // window before the new token: keys in ring slots
                           // first_slot, first_slot + 1, ... (mod keep + fine)
};

// The window of the step at `position` (local_len_at and its ring slots).
// Positions below 2^31 take 32-bit arithmetic.
TAO_DEV void step_window(long long position, int keep, int fine, int& n_old, int& first_slot) {
  const int L = keep + fine;
  if (position < 0x7FFFFFFFLL) {
    const int pos = (int)position;
    n_old = pos < L ? pos : keep + (pos - L) % fine;
    first_slot = (pos - n_old) % L;
  } else {
    n_old = local_len_at(position, keep, fine);
    first_slot = (int)((position - n_old) % L);
  }
}

// The fusion arguments of a step (copied out of the kernel arguments).
struct CombineArgs {
  const void* fa; const void* fb; int f_dtype;
  int64_t fa_s[3], fb_s[3];
  float gain;
};

template <typename P>
TAO_DEV CombineArgs combine_args(const P& p) {
  CombineArgs c;
  c.fa = p.fa;
  c.fb = p.fb;
  c.f_dtype = p.f_dtype;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    c.fa_s[i] = p.fa_s[i];
    c.fb_s[i] = p.fb_s[i];
  }
  c.gain = p.gain;
  return c;
}

// Fusion parameter element `off` of dtype FDT (a launch-time constant, so
// the loads of one channel's six parameters issue back to back).
template <int FDT>
TAO_DEV float param_at(const void* p, int64_t off) {
  if constexpr (FDT == TAO_FP32) return ((const float*)p)[off];
  else if constexpr (FDT == TAO_FP16) return (float)((const _Float16*)p)[off];
  else return bf2f(((const bf16_t*)p)[off]);
}

// Fine-read workgroup f: num[e] = h . G^T[e] for rows e in
// [f * kFineRows, (f + 1) * kFineRows) of the folded matrix gmat (this
// head's), thread (row tid / 8, part tid % 8); with gden (the fine read)
// workgroup 0 also writes den = r(h . g). h = r(softmax_D(raw_q)) with the
// exp correctly rounded in fp32. Wave 0 computes h on the bit-reversed
// layout (lane L holds channels fold_lane(L) + 64 k), so its sums are the
// fold order of the natural layout on DPP moves (no LDS round trips).
template <int D>
__device__ void fine_read(const bf16_t* rq, int f, float* frec, float* hq, const float* gmat,
                          const float* gden) {
  constexpr int DP = D / 8, PER = D / 64;
  const int tid = threadIdx.x, row = tid / 8, part = tid % 8;
  const int e = f * kFineRows + row;
  const bool with_den = gden != nullptr && f == 0;
  const float* grow = gmat + (size_t)e * D + part * DP;
  float gv[DP];
#pragma unroll
  for (int k = 0; k < DP; k += 4) {
    const float4 v = *(const float4*)(grow + k);
    gv[k] = v.x; gv[k + 1] = v.y; gv[k + 2] = v.z; gv[k + 3] = v.w;
  }
  if (tid < 64) {
    const int c0 = fold_lane(tid);
    float xr[PER], gd[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      xr[k] = bf2f(rq[c0 + 64 * k]);
      gd[k] = with_den ? gden[c0 + 64 * k] : 0.0f;
    }
    float top = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < PER; ++k) top = fmaxf(top, xr[k]);
    top = wave_fold_max(top);
    float ex[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) ex[k] = exp_cr(xr[k] - top);
    float s = ex[0];
#pragma unroll
    for (int k = 1; k < PER; ++k) s += ex[k];
    s = wave_fold_sum(s);
    float dsum = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const float hv = rbf(ex[k] / s);
      hq[c0 + 64 * k] = hv;
      dsum = k == 0 ? hv * gd[k] : fmaf(hv, gd[k], dsum);
    }
    if (with_den) {
      dsum = wave_fold_sum(dsum);
      if (tid == 0) st_agent(&frec[0], rbf(dsum));
    }
  }
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < DP; ++k) acc = fmaf(hq[part * DP + k], gv[k], acc);
  acc = row_sum<8>(acc);    // the xor-1, xor-2, xor-4 butterfly over the row's 8 parts
  if (part == 0) st_agent(&frec[kStepRec + e], acc);
}

// Workgroup j of one (request, head): j < NLOC local attention over keys
// [j*K, (j+1)*K) of the window (workgroup 0 also appends the new token to
// the ring), then NFINE fine-read workgroups (M > 0) and, with coarse_on,
// NFINE coarse-read workgroups. With `stamping` (diagnostic launches) a
// local unit returns the device clock after its scores, other units 0.
template <int D, int FDT>
__device__ unsigned long long units_body(const StepReq& q, int j, int M, int coarse_on, int keep,
                                         int fine, int slot_stride, StepSmem<D>& sm,
                                         const CombineArgs* fuse, int h, bool stamping = false) {
  using G = Geo<D>;
  constexpr int STRIDE = D + kStepRec;
  float* recs = q.recs;
  if (j >= G::NLOC + G::NFINE) {
    if (coarse_on)
      fine_read<D>(q.rq, j - G::NLOC - G::NFINE, recs + (G::NLOC + 1) * STRIDE, sm.wo[0],
                   q.coarse_g, nullptr);
    return 0ull;
  }
  if (j >= G::NLOC) {
    // Fine-read workgroup f; with `fuse`, its first kFineRows threads also
    // write the branch weights of channels f * kFineRows + tid (records
    // NLOC + 2 .. NLOC + 4), loading their operands before the read and
    // combining them after it.
    const int f = j - G::NLOC;
    const int e = f * kFineRows + (int)threadIdx.x;
    const bool weights = fuse != nullptr && (M > 0 || coarse_on) && threadIdx.x < kFineRows;
    float fq = 0.0f, fa3[3] = {}, fb3[3] = {};
    if (weights) {
      fq = bf2f(q.rq[e]);
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        fa3[i] = param_at<FDT>(fuse->fa, h * fuse->fa_s[0] + e * fuse->fa_s[1] + i * fuse->fa_s[2]);
        fb3[i] = param_at<FDT>(fuse->fb, h * fuse->fb_s[0] + e * fuse->fb_s[1] + i * fuse->fb_s[2]);
      }
    }
    if (M > 0)
      fine_read<D>(q.rq, f, recs + G::NLOC * STRIDE, sm.wo[0], q.fold_g, q.fold_den);
    if (weights) {
      const FuseWeights w = fuse_weights(fq, fa3, fb3, coarse_on, M > 0 ? 1 : 0);
      st_agent(recs + (G::NLOC + 2) * STRIDE + kStepRec + e, w.r0);
      st_agent(recs + (G::NLOC + 3) * STRIDE + kStepRec + e, w.r1);
      st_agent(recs + (G::NLOC + 4) * STRIDE + kStepRec + e, w.r2);
    }
    return 0ull;
  }
  float* rec = recs + j * (D + kStepRec);
  const int tid = threadIdx.x, chn = tid % G::CH, r = tid / G::CH;
  const int L = keep + fine;
  const int n_old = q.n_old, first_slot = q.first_slot;
  const int n = n_old + 1;
  const int k0 = j * G::KEYS;
  if (k0 >= n) {   // past the window: an empty record
    if (tid == 0) { st_agent(&rec[0], -__builtin_inff()); st_agent(&rec[1], 0.0f); }
    return 0ull;
  }
  // Issue every load first: the new token's row for the ring append
  // (workgroup 0), KPT key and value rows, the q chunk.
  static_assert(D <= kThreads, "one append element per thread");
  const bool appends = j == 0 && tid < D;
  bf16_t app_k = 0, app_v = 0, app_r = 0;
  if (appends) {
    app_k = q.k[tid];
    app_v = q.v[tid];
    app_r = q.rk[tid];
  }
  uint4 kraw[G::KPT], vraw[G::KPT];
#pragma unroll
  for (int i = 0; i < G::KPT; ++i) {
    const int key = k0 + r + i * G::ROWS;
    const bf16_t* krow = q.k;
    const bf16_t* vrow = q.v;
    if (key < n_old) {
      int slot = first_slot + key;
      slot = slot >= L ? slot - L : slot;
      const size_t off = (size_t)slot * slot_stride;
      krow = q.ring_k + off;
      vrow = q.ring_v + off;
    }
    kraw[i] = *(const uint4*)(krow + chn * 8);
    vraw[i] = *(const uint4*)(vrow + chn * 8);
  }
  float qv[8];
  unpack8(*(const uint4*)(q.q + chn * 8), qv);
  // Scores in log2 units (1/sqrt(D) and log2 e folded into one scale), each
  // reduced over its row's lanes; keys past the window score -inf.
  const float scale2 = (float)(1.4426950408889634 / __builtin_sqrt((double)D));
  float sc[G::KPT];
#pragma unroll
  for (int i = 0; i < G::KPT; ++i) {
    float kv[8];
    unpack8(kraw[i], kv);
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) part = fmaf(qv[e], kv[e], part);
    sc[i] = row_sum<G::CH>(part) * scale2;
    if (k0 + r + i * G::ROWS >= n) sc[i] = -__builtin_inff();
  }
  const unsigned long long scored = stamping ? __builtin_amdgcn_s_memrealtime() : 0ull;
  // Weights against the wave's maximum over its rows' keys (one value for
  // the whole wave, so no rescale inside it); a wave whose keys are all
  // past the window contributes nothing.
  float m = sc[0];
#pragma unroll
  for (int i = 1; i < G::KPT; ++i) m = fmaxf(m, sc[i]);
  m = wave_rows_max<G::CH>(m);
  float l = 0.0f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  if (m != -__builtin_inff()) {
#pragma unroll
    for (int i = 0; i < G::KPT; ++i) {
      const float w = __builtin_amdgcn_exp2f(sc[i] - m);   // 0 for a -inf score
      float vv[8];
      unpack8(vraw[i], vv);
      l += w;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(w, vv[e], acc[e]);
    }
  }
  // The wave's rows summed on lane swaps (no LDS), then the waves meet once
  // in LDS: a common maximum (wave 0 holds key k0 < n, so it is finite;
  // empty waves weigh exp2(-inf) = 0) and the rescaled sums in wave order.
  l = wave_rows_sum<G::CH>(l);
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = wave_rows_sum<G::CH>(acc[e]);
  const int wave = tid / 64, lane = tid % 64;
  if (lane < G::CH) {
    *(float4*)&sm.wo[wave][chn * 8] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *(float4*)&sm.wo[wave][chn * 8 + 4] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  if (lane == 0) { sm.wm[wave] = m; sm.wl[wave] = l; }
  __syncthreads();
  if (tid < D) {
    float top = sm.wm[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) top = fmaxf(top, sm.wm[w]);
    float sum = 0.0f, lsum = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = __builtin_amdgcn_exp2f(sm.wm[w] - top);
      sum = fmaf(f, sm.wo[w][tid], sum);
      lsum = fmaf(f, sm.wl[w], lsum);
    }
    st_agent(&rec[kStepRec + tid], sum);
    if (tid == 0) {
      st_agent(&rec[0], top);
      st_agent(&rec[1], lsum);
    }
  }
  if (appends) {
    // Append the new token at ring slot position % L, after this step's
    // reads: no key of this step's window occupies that slot (window
    // length n_old <= L - 1), and the stores are last so that no load
    // above waits for them.
    int slot = first_slot + n_old;
    slot = slot >= L ? slot - L : slot;
    const size_t off = (size_t)slot * slot_stride;
    q.ring_k[off + tid] = app_k;
    q.ring_v[off + tid] = app_v;
    q.ring_raw[off + tid] = app_r;
  }
  return scored;
}

// The units of one launch: per (batch, head) NLOC local-attention
// workgroups (the window split by keys), NFINE fine-read workgroups and,
// with coarse_on, NFINE coarse-read workgroups. Returns the (batch, head).
template <int D, int FDT>
__device__ int decode_units(const DecodeParams& p, int M, const CombineArgs& c,
                            bool stamping, unsigned long long& scored) {
  using G = Geo<D>;
  __shared__ StepSmem<D> sm;
  const int per_head = G::NLOC + G::NFINE * (p.coarse_on ? 2 : 1);
  int bh, j;
  xcd_unit(blockIdx.x, p.B * p.H, per_head, bh, j);
  const int b = bh / p.H, h = bh % p.H;
  StepReq q;
  q.q = p.q.p + b * p.q.sb + h * p.q.sh;
  q.k = p.k.p + b * p.k.sb + h * p.k.sh;
  q.v = p.v.p + b * p.v.sb + h * p.v.sh;
  q.rq = p.rq.p + b * p.rq.sb + h * p.rq.sh;
  q.rk = p.rk.p + b * p.rk.sb + h * p.rk.sh;
  const int L = p.keep + p.fine;
  const size_t ring0 = ((size_t)b * L * p.H + h) * D;
  q.ring_k = p.ring_k + ring0;
  q.ring_v = p.ring_v + ring0;
  q.ring_raw = p.ring_raw + ring0;
  q.fold_g = p.fold_g + (size_t)bh * D * D;
  q.fold_den = p.fold_den + (size_t)bh * D;
  q.coarse_g = p.coarse_g ? p.coarse_g + (size_t)bh * D * D : nullptr;
  q.recs = p.parts + (size_t)bh * step_floats(D, p.sel_cap);
  if (p.pos_hint >= 0) {
    q.n_old = p.win_n_old;
    q.first_slot = p.win_first;
  } else {
    step_window(p.header[0], p.keep, p.fine, q.n_old, q.first_slot);
  }
  scored = units_body<D, FDT>(q, j, M, p.coarse_on, p.keep, p.fine, p.H * D, sm, &c, h,
                              stamping);
  return bh;
}

// The merge of one (request, head)'s records into its output channels and
// the fusion epilogue. The batched step runs it as its own kernel, one
// workgroup per (request, head, kCombineCols channels).
constexpr int kCombineCols = 32;

// COLS channels (from chunk * COLS) of one (request, head); the first COLS
// threads own one channel each and the others return at once. An owner
// loads every record's maximum and weight sum (m, l) itself (one address per
// wave, so one request per wave) together with its channel's local sums,
// the fine and coarse records and the fusion operands: one round of loads,
// then registers only (no LDS, no barrier). Each channel's local numerator
// sums the records in index order, so the merge gives the same bits for any
// COLS: the single-request step (COLS = D) and the batched combine kernel
// (COLS = kCombineCols) agree exactly. AGENT: the records were published by
// other workgroups of the same launch (device-coherent loads). FDT: the
// fusion parameters' dtype. Empty records (past the window) hold m = -inf
// and l = 0, so they take part in the maxima and weights as exp2(-inf) = 0;
// record 0 always holds the new token, so the common maximum is finite.
template <int D, int COLS, bool AGENT, int FDT, bool WEIGHTED>
__device__ void combine_body(const float* recs, const bf16_t* rq, bf16_t* out, int h, int chunk,
                             int M, int coarse_on, const CombineArgs& c) {
  using Gm = Geo<D>;
  constexpr int STRIDE = D + kStepRec;
  constexpr int NLOC = Gm::NLOC;
  const int tid = threadIdx.x;
  if (tid >= COLS) return;
  const int d = chunk * COLS + tid;
  auto ld = [](const float* x) __attribute__((always_inline)) {
    return AGENT ? ld_agent(x) : *x;
  };

  float m_j[NLOC], l_j[NLOC], o_j[NLOC];
#pragma unroll
  for (int j = 0; j < NLOC; ++j) {
    m_j[j] = ld(recs + j * STRIDE);
    l_j[j] = ld(recs + j * STRIDE + 1);
    o_j[j] = ld(recs + j * STRIDE + kStepRec + d);
  }
  // The fine, coarse and weight records are loaded whatever M and
  // coarse_on say (every step's scratch holds them), so that no load waits
  // behind a branch; values of records this step did not write are only
  // ever discarded by selects below, never multiplied.
  const float den_r = ld(recs + NLOC * STRIDE);
  const float num_r = ld(recs + NLOC * STRIDE + kStepRec + d);
  const float craw_r = ld(recs + (NLOC + 1) * STRIDE + kStepRec + d);
  float qx = 0.0f, fa3[3] = {}, fb3[3] = {};
  FuseWeights wts{};
  if (WEIGHTED) {
    wts.r0 = ld(recs + (NLOC + 2) * STRIDE + kStepRec + d);
    wts.r1 = ld(recs + (NLOC + 3) * STRIDE + kStepRec + d);
    wts.r2 = ld(recs + (NLOC + 4) * STRIDE + kStepRec + d);
  } else {
    qx = bf2f(rq[d]);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      fa3[i] = param_at<FDT>(c.fa, h * c.fa_s[0] + d * c.fa_s[1] + i * c.fa_s[2]);
      fb3[i] = param_at<FDT>(c.fb, h * c.fb_s[0] + d * c.fb_s[1] + i * c.fb_s[2]);
    }
  }
  float top = m_j[0];
#pragma unroll
  for (int j = 1; j < NLOC; ++j) top = fmaxf(top, m_j[j]);
  float den_local = 0.0f, nl = 0.0f;
#pragma unroll
  for (int j = 0; j < NLOC; ++j) {
    const float w = __builtin_amdgcn_exp2f(m_j[j] - top);
    den_local = fmaf(w, l_j[j], den_local);
    nl += l_j[j] > 0.0f ? w * o_j[j] : 0.0f;
  }
  const float local = rbf(nl / den_local);
  bf16_t result;
  if (M > 0 || coarse_on) {
    const float fine_v = M > 0 ? rbf(rbf(num_r) / den_r) : 0.0f;
    const float coarse_v = coarse_on ? rbf(craw_r) : 0.0f;
    if (!WEIGHTED) wts = fuse_weights(qx, fa3, fb3, coarse_on ? 1 : 0, M > 0 ? 1 : 0);
    result = fuse_mix(wts, local, coarse_v, fine_v, c.gain);
  } else {
    result = f2bf(local);
  }
  out[d] = result;
}

// The single-launch step: the units of every (batch, head) publish their
// records with device-coherent stores, wait for them to complete and count
// themselves in on the head's arrival counter; the head's last workgroup
// merges the records and applies the fusion for all D channels. The
// counters (p.counters: one per head, one for the launch) start at zero and
// are reset by their last arrival, so every step starts from zero. The head that completes last advances the cursor in header[0].
template <int D, int FDT>
__global__ __launch_bounds__(kThreads) void decode_step_kernel(DecodeParams p, int M) {
  __shared__ int last;
  // Diagnostic clock stamps (p.stamps is null in production launches).
  const bool stamping = p.stamps != nullptr;
  const unsigned long long t0 = stamping ? __builtin_amdgcn_s_memrealtime() : 0ull;
  const int per_head = Geo<D>::NLOC + Geo<D>::NFINE * (p.coarse_on ? 2 : 1);
  const CombineArgs c = combine_args(p);
  unsigned long long t1;
  const int bh = decode_units<D, FDT>(p, M, c, stamping, t1);
  const unsigned long long t2 = stamping ? __builtin_amdgcn_s_memrealtime() : 0ull;
  float* recs = p.parts + (size_t)bh * step_floats(D, p.sel_cap);
  unsigned* head_count = p.counters + (size_t)bh * kCounterStride;
  // Release of the records at agent scope without an L2 write-back: every
  // record was stored with an agent-scope (write-through) store, so once
  // each thread's stores are acknowledged (vmcnt 0) an agent-scope load on
  // any XCD returns them. A workgroup-scope fence does not wait for them
  // (gfx950 lowers it to an LDS wait), so every wave waits here, before the
  // barrier that orders its stores before thread 0's arrival count.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const unsigned long long t3 = stamping ? __builtin_amdgcn_s_memrealtime() : 0ull;
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(head_count, 1u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) == (unsigned)per_head - 1u;
  __syncthreads();
  const unsigned long long t4 = stamping ? __builtin_amdgcn_s_memrealtime() : 0ull;
  // The unit's stamp frame: its five stamps, the merge's end (the head's
  // last arrival only), its identity and its placement.
  auto stamp = [&](unsigned long long t5) __attribute__((always_inline)) {
    if (!stamping || threadIdx.x != 0) return;
    int u, j;
    xcd_unit(blockIdx.x, p.B * p.H, per_head, u, j);
    const unsigned xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20);   // XCC_ID[3:0]
    ulonglong4* f = (ulonglong4*)(p.stamps + (size_t)blockIdx.x * kStampWords);
    f[0] = make_ulonglong4(t0, t1 ? t1 : t2, t2, t3);   // fine units: no scores stamp
    f[1] = make_ulonglong4(t4, t5, ((unsigned long long)j << 32) | (unsigned)u,
                           ((unsigned long long)xcc << 32) | __smid());
  };
  if (!last) {
    stamp(0ull);
    return;
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(head_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int b = bh / p.H, h = bh % p.H;
  combine_body<D, D, true, FDT, true>(recs, p.rq.p + b * p.rq.sb + h * p.rq.sh,
                                      p.out + b * p.out_sb + h * p.out_sh, h, 0, M, p.coarse_on,
                                      c);
  if (p.pos_hint >= 0) {
    // The stream position advances once per step (graph replays read it).
    // With the cursor given by the host no workgroup reads it, so head 0's
    // merge stores the next one.
    if (bh == 0 && threadIdx.x == 0) p.header[0] = p.pos_hint + 1;
  } else if (threadIdx.x == 0) {
    // Every workgroup of the launch read the cursor before it arrived: the
    // last head advances it.
    unsigned* all_count = p.counters + (size_t)p.B * p.H * kCounterStride;
    if (__hip_atomic_fetch_add(all_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        (unsigned)(p.B * p.H) - 1u) {
      __hip_atomic_store(all_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      p.header[0] = p.header[0] + 1;
    }
  }
  if (stamping) stamp(__builtin_amdgcn_s_memrealtime());
}

// Batched step over R requests (one state each, batch 1): request r's token
// rows are batch row r of the operands, its buffers come from the device
// table, its cursor from its header[0] and its route size from header[1].
// Local workgroup 0 of each (request, head) leaves M and coarse_on in its
// record for kernel B, whose workgroup (request, head 0, chunk 0) advances
// header[0].
template <int D>
__global__ __launch_bounds__(kThreads) void batch_units_kernel(BatchStepParams p) {
  using G = Geo<D>;
  __shared__ StepSmem<D> sm;
  const int per_head = G::NLOC + G::NFINE * (p.coarse_values ? 2 : 1);
  int rh, j;
  xcd_unit(blockIdx.x, p.R * p.H, per_head, rh, j);
  const int r = rh / p.H, h = rh % p.H;
  const BatchReq& t = p.table[r];
  StepReq q;
  q.q = p.q.p + r * p.q.sb + h * p.q.sh;
  q.k = p.k.p + r * p.k.sb + h * p.k.sh;
  q.v = p.v.p + r * p.v.sb + h * p.v.sh;
  q.rq = p.rq.p + r * p.rq.sb + h * p.rq.sh;
  q.rk = p.rk.p + r * p.rk.sb + h * p.rk.sh;
  q.ring_k = t.ring_k + (size_t)h * D;
  q.ring_v = t.ring_v + (size_t)h * D;
  q.ring_raw = t.ring_raw + (size_t)h * D;
  q.fold_g = t.fold_g + (size_t)h * D * D;
  q.fold_den = t.fold_den + (size_t)h * D;
  q.coarse_g = t.coarse_g ? t.coarse_g + (size_t)h * D * D : nullptr;
  q.recs = t.parts + (size_t)h * step_floats(D, 0);
  const long long position = t.header[0];
  step_window(position, p.keep, p.fine, q.n_old, q.first_slot);
  const long long fines = fines_before(position, p.keep, p.fine);
  const int M = fines > 0 ? (int)t.header[1] : 0;
  const int coarse_on = q.coarse_g != nullptr && fines >= p.group;
  if (j == 0 && threadIdx.x == 0) {
    q.recs[2] = (float)M;
    q.recs[3] = (float)coarse_on;
  }
  units_body<D, TAO_BF16>(q, j, M, coarse_on, p.keep, p.fine, p.H * D, sm, nullptr, h);
}

template <int D, int FDT>
__global__ __launch_bounds__(kThreads) void batch_combine_kernel(BatchStepParams p) {
  constexpr int CHUNKS = D / kCombineCols;
  int rh, chunk;
  xcd_unit(blockIdx.x, p.R * p.H, CHUNKS, rh, chunk);
  const int r = rh / p.H, h = rh % p.H;
  const BatchReq& t = p.table[r];
  const float* recs = t.parts + (size_t)h * step_floats(D, 0);
  const int M = (int)recs[2];
  const int coarse_on = recs[3] != 0.0f;
  const CombineArgs c = combine_args(p);
  combine_body<D, kCombineCols, false, FDT, false>(recs, p.rq.p + r * p.rq.sb + h * p.rq.sh,
                                       p.out + r * p.out_sb + h * p.out_sh, h, chunk, M,
                                       coarse_on, c);
  if (h == 0 && chunk == 0 && threadIdx.x == 0) t.header[0] = t.header[0] + 1;
}

// Fold: one workgroup per (batch, head, ROWS rows of G^T). Thread (row r,
// chunk c) accumulates G^T[e0 + r][8c .. 8c + 8) over the selected slots in
// slot order (fp32), with w_m[d] = pw[page(m)][d] * sw[m][d]. A refresh is a
// chain of memory latencies, so every load of a stage is issued before any
// of them is used: the stage's ids, then its weights (staged in LDS once per
// workgroup) together with all its C rows (kFoldStage slots).
constexpr int kFoldStage = 36;

template <int D>
__global__ __launch_bounds__(kThreads) void fold_kernel(FoldParams p) {
  constexpr int CH = D / 8, ROWS = kThreads / CH, CHUNKS = D / ROWS, U = kFoldStage;
  constexpr int WPT = (U * CH + kThreads - 1) / kThreads;   // weight chunks per thread
  __shared__ float wts[U][D];
  __shared__ int ids[U];
  if (gate_closed(p.gate)) return;   // uniform: every thread reads one header word
  int bh, e_chunk;
  xcd_unit(blockIdx.x, p.B * p.H, CHUNKS, bh, e_chunk);
  const int e0 = e_chunk * ROWS;
  const int tid = threadIdx.x, c = tid % CH, r = tid / CH;
  const int e = e0 + r;
  const int32_t* sel = p.sel + (size_t)bh * p.sel_cap;
  const bf16_t* bank = p.bank + (size_t)bh * p.fine_cap * D * D;
  const bf16_t* sw = p.sw + (size_t)bh * p.fine_cap * D;
  const bf16_t* pw = p.pw + (size_t)bh * p.page_cap * D;
  float acc[8], den[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) { acc[k] = 0.0f; den[k] = 0.0f; }
  for (int s0 = 0; s0 < p.M; s0 += U) {
    const int staged = min(U, p.M - s0);
    __syncthreads();                  // the previous stage is consumed
    if (tid < staged) ids[tid] = sel[s0 + tid];
    __syncthreads();
    uint4 wp[WPT], ws[WPT], cv[U];
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
      const int i = tid + k * kThreads;
      if (i < staged * CH) {
        const int id = ids[i / CH], cc = i % CH;
        wp[k] = *(const uint4*)(pw + (size_t)(id / p.group) * D + cc * 8);
        ws[k] = *(const uint4*)(sw + (size_t)id * D + cc * 8);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int m = min(u, staged - 1);
      cv[u] = *(const uint4*)(bank + ((size_t)ids[m] * D + e) * D + c * 8);
    }
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
      const int i = tid + k * kThreads;
      if (i < staged * CH) {
        float pf[8], sf[8];
        unpack8(wp[k], pf);
        unpack8(ws[k], sf);
#pragma unroll
        for (int j = 0; j < 8; ++j) wts[i / CH][(i % CH) * 8 + j] = pf[j] * sf[j];
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (u < staged) {
        float cf[8];
        unpack8(cv[u], cf);
        const float4 wa = *(const float4*)&wts[u][c * 8];
        const float4 wb = *(const float4*)&wts[u][c * 8 + 4];
        const float w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          acc[k] = fmaf(w[k], cf[k], acc[k]);
          den[k] += w[k];
        }
      }
    }
  }
  float* grow = p.fold_g + ((size_t)bh * D + e) * D + c * 8;
  *(float4*)grow = make_float4(acc[0], acc[1], acc[2], acc[3]);
  *(float4*)(grow + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
  if (e == 0) {
    float* dg = p.fold_den + (size_t)bh * D + c * 8;
    *(float4*)dg = make_float4(den[0], den[1], den[2], den[3]);
    *(float4*)(dg + 4) = make_float4(den[4], den[5], den[6], den[7]);
  }
}

__global__ __launch_bounds__(kThreads) void ring_append_kernel(AppendParams p) {
  // grid: (count, B*H); copies D elements of k, v, raw_k per (token, b, h).
  const int t = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int slot = (int)((p.pos + t) % p.L);
  const int tok = p.first + t;
  const size_t dst = (((size_t)b * p.L + slot) * p.H + h) * p.D;
  for (int d = threadIdx.x; d < p.D; d += kThreads) {
    p.ring_k[dst + d] = p.k.p[b * p.k.sb + tok * p.k.st + h * p.k.sh + d];
    p.ring_v[dst + d] = p.v.p[b * p.v.sb + tok * p.v.st + h * p.v.sh + d];
    p.ring_raw[dst + d] = p.rk.p[b * p.rk.sb + tok * p.rk.st + h * p.rk.sh + d];
  }
}

// The same copy with one thread per 16-byte chunk of a row (rows of the
// three operands 16-byte aligned), grid-strided over (token, b, h, chunk).
__global__ __launch_bounds__(kThreads) void ring_append_vec_kernel(AppendParams p) {
  const int cpr = p.D / 8;
  const long long n = (long long)p.count * p.B * p.H * cpr;
  for (long long i = (long long)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (long long)gridDim.x * kThreads) {
    const int c = (int)(i % cpr);
    long long r = i / cpr;
    const int h = (int)(r % p.H);
    r /= p.H;
    const int b = (int)(r % p.B);
    const int t = (int)(r / p.B);
    const int slot = (int)((p.pos + t) % p.L);
    const long long tok = p.first + t;
    const size_t dst = (((size_t)b * p.L + slot) * p.H + h) * p.D + 8 * c;
    *(uint4*)(p.ring_k + dst) = *(const uint4*)(p.k.p + b * p.k.sb + tok * p.k.st + h * p.k.sh + 8 * c);
    *(uint4*)(p.ring_v + dst) = *(const uint4*)(p.v.p + b * p.v.sb + tok * p.v.st + h * p.v.sh + 8 * c);
    *(uint4*)(p.ring_raw + dst) =
        *(const uint4*)(p.rk.p + b * p.rk.sb + tok * p.rk.st + h * p.rk.sh + 8 * c);
  }
}

}  // namespace

// Calls f(std::integral_constant<int, FDT>{}) for the fusion dtype.
template <typename F>
hipError_t with_fusion_dtype(int dtype, F&& f) {
  switch (dtype) {
    case TAO_BF16: f(std::integral_constant<int, TAO_BF16>{}); break;
    case TAO_FP32: f(std::integral_constant<int, TAO_FP32>{}); break;
    case TAO_FP16: f(std::integral_constant<int, TAO_FP16>{}); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

namespace {

// The diagnostic stamp recorder (host state; see step_stamps_set).
struct StampRecorder {
  unsigned long long* buf = nullptr;
  long long frames = 0, frame_words = 0, launches = 0;
};
StampRecorder g_stamps;

}  // namespace

int step_stamps_set(void* buf, long long frames, long long frame_words) {
  if (buf && (frames <= 0 || frame_words < kStampWords)) return -1;
  g_stamps.buf = (unsigned long long*)buf;
  g_stamps.frames = buf ? frames : 0;
  g_stamps.frame_words = buf ? frame_words : 0;
  g_stamps.launches = 0;
  return 0;
}

long long step_stamps_count() { return g_stamps.launches; }

namespace {

// Stamp frame of the next eager launch of `units` workgroups (graph
// captures and device-cursor steps record none), or null.
unsigned long long* next_stamp_frame(const DecodeParams& p, unsigned units) {
  if (!g_stamps.buf || p.pos_hint < 0) return nullptr;
  if ((long long)units * kStampWords > g_stamps.frame_words) return nullptr;
  unsigned long long* f =
      g_stamps.buf + (size_t)(g_stamps.launches % g_stamps.frames) * g_stamps.frame_words;
  ++g_stamps.launches;
  return f;
}

}  // namespace

hipError_t launch_decode_step(const DecodeParams& p, int head_dim, int M, hipStream_t s) {
  if (M < 0 || M > p.sel_cap) return hipErrorInvalidValue;
  if (p.keep + p.fine > kMaxWindow) return hipErrorInvalidValue;
  if (p.coarse_on && !p.coarse_g) return hipErrorInvalidValue;
  if (!p.parts || !p.counters) return hipErrorInvalidValue;
  if (head_dim != 128 && head_dim != 64) return hipErrorInvalidValue;
  DecodeParams q = p;
  if (q.pos_hint >= 0) {
    // The window of this step, from the cursor the host passes.
    const long long L = q.keep + q.fine;
    const long long n_old = q.pos_hint < L ? q.pos_hint : q.keep + (q.pos_hint - L) % q.fine;
    q.win_n_old = (int)n_old;
    q.win_first = (int)((q.pos_hint - n_old) % L);
  }
  const int per_head = local_units(head_dim) + fine_units(head_dim) * (q.coarse_on ? 2 : 1);
  const dim3 units((unsigned)(q.B * q.H * per_head));
  q.stamps = next_stamp_frame(q, units.x);
  return with_fusion_dtype(q.f_dtype, [&](auto fdt) {
    constexpr int FDT = decltype(fdt)::value;
    if (head_dim == 128)
      hipLaunchKernelGGL((decode_step_kernel<128, FDT>), units, dim3(kThreads), 0, s, q, M);
    else
      hipLaunchKernelGGL((decode_step_kernel<64, FDT>), units, dim3(kThreads), 0, s, q, M);
  });
}

hipError_t launch_batch_step(const BatchStepParams& p, int head_dim, hipStream_t s) {
  if (p.R <= 0) return hipSuccess;
  if (p.keep + p.fine > kMaxWindow) return hipErrorInvalidValue;
  if (head_dim != 128 && head_dim != 64) return hipErrorInvalidValue;
  const int per_head = local_units(head_dim) + fine_units(head_dim) * (p.coarse_values ? 2 : 1);
  const dim3 units((unsigned)(p.R * p.H * per_head));
  const dim3 cols((unsigned)(p.R * p.H * (head_dim / kCombineCols)));
  return with_fusion_dtype(p.f_dtype, [&](auto fdt) {
    constexpr int FDT = decltype(fdt)::value;
    if (head_dim == 128) {
      hipLaunchKernelGGL(batch_units_kernel<128>, units, dim3(kThreads), 0, s, p);
      hipLaunchKernelGGL((batch_combine_kernel<128, FDT>), cols, dim3(kThreads), 0, s, p);
    } else {
      hipLaunchKernelGGL(batch_units_kernel<64>, units, dim3(kThreads), 0, s, p);
      hipLaunchKernelGGL((batch_combine_kernel<64, FDT>), cols, dim3(kThreads), 0, s, p);
    }
  });
}

hipError_t launch_fold(const FoldParams& p, int head_dim, hipStream_t s) {
  if (p.M < 0 || p.M > p.sel_cap) return hipErrorInvalidValue;
  if (head_dim == 128) {
    constexpr int CHUNKS = 128 / (kThreads / 16);
    hipLaunchKernelGGL(fold_kernel<128>, dim3((unsigned)(p.B * p.H * CHUNKS)), dim3(kThreads),
                       0, s, p);
  } else if (head_dim == 64) {
    constexpr int CHUNKS = 64 / (kThreads / 8);
    hipLaunchKernelGGL(fold_kernel<64>, dim3((unsigned)(p.B * p.H * CHUNKS)), dim3(kThreads),
                       0, s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_ring_append(const AppendParams& p, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  auto aligned = [](const TokView& t) {
    return ((uintptr_t)t.p & 15) == 0 && t.sb % 8 == 0 && t.st % 8 == 0 && t.sh % 8 == 0;
  };
  if (p.D % 8 == 0 && aligned(p.k) && aligned(p.v) && aligned(p.rk)) {
    const long long chunks = (long long)p.count * p.B * p.H * (p.D / 8);
    const long long blocks = std::min<long long>((chunks + kThreads - 1) / kThreads, 4096);
    hipLaunchKernelGGL(ring_append_vec_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL(ring_append_kernel, dim3((unsigned)p.count, (unsigned)(p.B * p.H)),
                       dim3(kThreads), 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace tao
