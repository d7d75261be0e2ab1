// Fused single-token decode step for gfx950.
//
// Two launches per new token (replace, per request x layer, the reference's
// q1 page-memo region tao_stream.py:418-433 + query_fresh_fine.py:8-75, the
// local SDPA flash_attention.py:25-29 over torch.cat'ed K/V
// tao_stream.py:927-930, and the fusion kernels fusion_pointwise.py:10-117):
//
// decode_units_kernel: per (batch, head) local_units(D) + kFineUnits
//   independent workgroups.
//   local workgroup j : keys [j*D/2, (j+1)*D/2) of the exact window (K and
//                       V rows from the ring, or the new token), one online
//                       softmax per key row, merged into a record (m, l,
//                       o[D]); workgroup 0 also appends the new token to the
//                       ring. Its only scalar input is the cursor (a kernel
//                       argument in eager launches, header[0] in graphs).
//   fine workgroup w  : selected slots m = w, w + kFineUnits, ... Each slot
//                       streams its D x D bf16 C^T matrix (16-byte loads, 1
//                       KB per wave instruction) through two register
//                       stages, so the next slot's loads are in flight while
//                       the current one is contracted with
//                       ch = r(r(h*pw[page]) * sw[fine]) (h computed once).
//                       Writes a record num[D] and r(sum_d ch) per slot.
// decode_combine_kernel: one workgroup per (batch, head, 32 channels)
//   merges the records in a fixed order, den = r(sum_m r(sum_d ch)) in
//   butterfly order over the slots, fine = r(r(num)/den), applies the fusion
//   epilogue and advances header[0] (the stream position), so the pair can
//   be replayed from a hipGraph.
// The kernel boundary publishes the records across the eight XCD L2 caches:
// a device-scope release fence per workgroup (last-block combine) costs far
// more than the second launch on this part.
#include "tao_launch.h"
#include "tao_common.h"
#include "tao_fusion.h"

namespace tao {
namespace {

constexpr int kMaxFinesPerWG = (512 + kFineUnits - 1) / kFineUnits;

template <int D>
struct Geo {
  static constexpr int CH = D / 8;                 // 16-byte chunks per row
  static constexpr int ROWS = kThreads / CH;       // rows per load pass
  static constexpr int RPT = D / ROWS;             // uint4 per thread per C^T
  static constexpr int KEYS = D / 2;               // keys per local workgroup
  static constexpr int KPT = KEYS / ROWS;          // key rows per thread
  static constexpr int PER = D / 64;               // channels per lane (wave 0)
  static constexpr int RED = ROWS > CH ? ROWS : CH;
  static constexpr int NLOC = local_units(D);
};

template <int D>
struct StepSmem {
  float chb[2][D];               // ch of the current / previous fine
  float red[Geo<D>::RED][D];     // cross-thread reductions
  float rm[Geo<D>::ROWS], rl[Geo<D>::ROWS];
  int ids[kMaxFinesPerWG];
};

TAO_DEV void unpack8(const uint4& u, float out[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

// Sum over the CH consecutive lanes that share one row.
template <int CH>
TAO_DEV float group_sum(float v) {
#pragma unroll
  for (int off = CH / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int D>
__device__ void local_workgroup(const DecodeParams& p, int b, int h, int j, float* rec,
                                StepSmem<D>& sm) {
  using G = Geo<D>;
  const int tid = threadIdx.x, chn = tid % G::CH, r = tid / G::CH;
  const int L = p.keep + p.fine;
  const long long position = p.pos_hint >= 0 ? p.pos_hint : p.header[0];
  const int n_old = local_len_at(position, p.keep, p.fine);
  const int n = n_old + 1;
  const int first_slot = (int)((position - n_old) % L);
  const bf16_t* kn = p.k.p + b * p.k.sb + h * p.k.sh;
  const bf16_t* vn = p.v.p + b * p.v.sb + h * p.v.sh;
  const int k0 = j * G::KEYS;
  if (k0 >= n) {   // past the window: an empty record
    if (tid == 0) { rec[0] = -__builtin_inff(); rec[1] = 0.0f; }
    return;
  }
  // Issue every load first: KPT key and value rows, the q chunk.
  uint4 kraw[G::KPT], vraw[G::KPT];
#pragma unroll
  for (int i = 0; i < G::KPT; ++i) {
    const int key = k0 + r + i * G::ROWS;
    const bf16_t* krow = kn;
    const bf16_t* vrow = vn;
    if (key < n_old) {
      int slot = first_slot + key;
      slot = slot >= L ? slot - L : slot;
      const size_t off = (((size_t)b * L + slot) * p.H + h) * D;
      krow = p.ring_k + off;
      vrow = p.ring_v + off;
    }
    kraw[i] = *(const uint4*)(krow + chn * 8);
    vraw[i] = *(const uint4*)(vrow + chn * 8);
  }
  float qv[8];
  unpack8(*(const uint4*)(p.q.p + b * p.q.sb + h * p.q.sh + chn * 8), qv);
  if (j == 0) {
    // Append the new token at slot position % L. No key of this step's
    // window occupies that slot (window length n_old <= L - 1).
    int slot = first_slot + n_old;
    slot = slot >= L ? slot - L : slot;
    const size_t off = (((size_t)b * L + slot) * p.H + h) * D;
    const bf16_t* rk = p.rk.p + b * p.rk.sb + h * p.rk.sh;
    for (int d = tid; d < D; d += kThreads) {
      p.ring_k[off + d] = kn[d];
      p.ring_v[off + d] = vn[d];
      p.ring_raw[off + d] = rk[d];
    }
  }
  const float scale = (float)(1.0 / __builtin_sqrt((double)D));
  float m = -__builtin_inff(), l = 0.0f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
  for (int i = 0; i < G::KPT; ++i) {
    float kv[8];
    unpack8(kraw[i], kv);
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) part = fmaf(qv[e], kv[e], part);
    const float s = group_sum<G::CH>(part) * scale;
    if (k0 + r + i * G::ROWS < n) {
      const float mn = fmaxf(m, s);
      const float keep = __expf(m - mn);
      const float w = __expf(s - mn);
      float vv[8];
      unpack8(vraw[i], vv);
      l = fmaf(l, keep, w);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(acc[e], keep, w * vv[e]);
      m = mn;
    }
  }
  // Merge the per-row online softmax states.
  if (chn == 0) { sm.rm[r] = m; sm.rl[r] = l; }
  __syncthreads();
  float top = -__builtin_inff();
#pragma unroll
  for (int rr = 0; rr < G::ROWS; ++rr)
    if (sm.rl[rr] > 0.0f) top = fmaxf(top, sm.rm[rr]);
  const float f = l > 0.0f ? __expf(m - top) : 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) sm.red[r][chn * 8 + e] = acc[e] * f;
  __syncthreads();
  if (tid < D) {
    float s = 0.0f;
    for (int rr = 0; rr < G::ROWS; ++rr) s += sm.red[rr][tid];
    rec[kStepRec + tid] = s;
  }
  if (tid == 0) {
    float lsum = 0.0f;
    for (int rr = 0; rr < G::ROWS; ++rr)
      if (sm.rl[rr] > 0.0f) lsum = fmaf(__expf(sm.rm[rr] - top), sm.rl[rr], lsum);
    rec[0] = top;
    rec[1] = lsum;
  }
}

template <int D>
struct FineRegs {
  uint4 x[Geo<D>::RPT];
  float pw[Geo<D>::PER], sw[Geo<D>::PER];   // wave 0
};

// Issue every load of this workgroup's k-th fine (no waits).
template <int D>
TAO_DEV void load_fine(const DecodeParams& p, int bh, int id, FineRegs<D>& x) {
  using G = Geo<D>;
  const int tid = threadIdx.x, chn = tid % G::CH, r = tid / G::CH;
  const bf16_t* cmat = p.bank + ((size_t)bh * p.fine_cap + id) * D * D;
#pragma unroll
  for (int i = 0; i < G::RPT; ++i)
    x.x[i] = *(const uint4*)(cmat + (size_t)(r + i * G::ROWS) * D + chn * 8);
  if (tid < 64) {
    const bf16_t* pw = p.pw + ((size_t)bh * p.page_cap + id / p.group) * D;
    const bf16_t* sw = p.sw + ((size_t)bh * p.fine_cap + id) * D;
#pragma unroll
    for (int k = 0; k < G::PER; ++k) {
      x.pw[k] = bf2f(pw[tid + 64 * k]);
      x.sw[k] = bf2f(sw[tid + 64 * k]);
    }
  }
}

template <int D>
__device__ void fine_workgroup(const DecodeParams& p, int b, int h, int w, int M, float* rec,
                               float* dens, StepSmem<D>& sm) {
  using G = Geo<D>;
  const int tid = threadIdx.x, chn = tid % G::CH, r = tid / G::CH;
  const int bh = b * p.H + h;
  const int nfine = M > w ? (M - 1 - w) / kFineUnits + 1 : 0;
  const int32_t* sel = p.sel + (size_t)bh * p.sel_cap;
  for (int k = tid; k < nfine; k += kThreads) sm.ids[k] = sel[w + k * kFineUnits];
  const bf16_t* rq = p.rq.p + b * p.rq.sb + h * p.rq.sh;
  float xr[G::PER];
  if (tid < 64) {
#pragma unroll
    for (int k = 0; k < G::PER; ++k) xr[k] = bf2f(rq[tid + 64 * k]);
  }
  __syncthreads();
  FineRegs<D> A, B;
  if (nfine > 0) load_fine<D>(p, bh, sm.ids[0], A);
  if (nfine > 1) load_fine<D>(p, bh, sm.ids[1], B);
  // h = r(softmax_D(raw_q)) by wave 0 (exp correctly rounded in fp32),
  // under the first loads.
  float hq[G::PER];
  if (tid < 64) {
    float top = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < G::PER; ++k) top = fmaxf(top, xr[k]);
    top = wave_max(top);
    float e[G::PER];
#pragma unroll
    for (int k = 0; k < G::PER; ++k) e[k] = exp_cr(xr[k] - top);
    float s = e[0];
#pragma unroll
    for (int k = 1; k < G::PER; ++k) s += e[k];
    s = wave_sum_fold(s);
#pragma unroll
    for (int k = 0; k < G::PER; ++k) hq[k] = rbf(e[k] / s);
  }
  float part[G::RPT];
#pragma unroll
  for (int i = 0; i < G::RPT; ++i) part[i] = 0.0f;
  auto consume = [&](int k, const FineRegs<D>& x) {
    float* chb = sm.chb[k & 1];
    if (tid < 64) {
      float csum = 0.0f;
#pragma unroll
      for (int q = 0; q < G::PER; ++q) {
        const float hv = rbf(hq[q] * x.pw[q]);
        const float ch = rbf(hv * x.sw[q]);
        chb[tid + 64 * q] = ch;
        csum = q == 0 ? ch : csum + ch;   // PER <= 2: fold of the lane pair
      }
      csum = wave_sum_fold(csum);
      if (tid == 0) dens[w + k * kFineUnits] = rbf(csum);
    }
    __syncthreads();
    float chv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) chv[q] = chb[chn * 8 + q];
#pragma unroll
    for (int i = 0; i < G::RPT; ++i) {
      float cf[8];
      unpack8(x.x[i], cf);
#pragma unroll
      for (int q = 0; q < 8; ++q) part[i] = fmaf(chv[q], cf[q], part[i]);
    }
  };
  // Two register stages: fine k + 1 is in flight while fine k is consumed.
  for (int k = 0; k < nfine; k += 2) {
    consume(k, A);
    if (k + 2 < nfine) load_fine<D>(p, bh, sm.ids[k + 2], A);
    if (k + 1 >= nfine) break;
    consume(k + 1, B);
    if (k + 3 < nfine) load_fine<D>(p, bh, sm.ids[k + 3], B);
  }
  // Record: sum the partial dots over the CH chunks of each row.
#pragma unroll
  for (int i = 0; i < G::RPT; ++i) sm.red[chn][r + i * G::ROWS] = part[i];
  __syncthreads();
  if (tid < D) {
    float s = 0.0f;
    for (int cc = 0; cc < G::CH; ++cc) s += sm.red[cc][tid];
    rec[kStepRec + tid] = s;
  }
}

// Kernel A: independent workgroups, no cross-workgroup communication.
template <int D>
__global__ __launch_bounds__(kThreads) void decode_units_kernel(DecodeParams p, int M) {
  using G = Geo<D>;
  __shared__ StepSmem<D> sm;
  constexpr int PER_HEAD = G::NLOC + kFineUnits;
  const int bh = blockIdx.x / PER_HEAD;
  const int role = blockIdx.x % PER_HEAD;
  const int b = bh / p.H, h = bh % p.H;
  float* recs = p.parts + (size_t)bh * step_floats(D, p.sel_cap);
  float* dens = recs + PER_HEAD * (D + kStepRec);
  if (role < G::NLOC)
    local_workgroup<D>(p, b, h, role, recs + role * (D + kStepRec), sm);
  else
    fine_workgroup<D>(p, b, h, role - G::NLOC, M, recs + role * (D + kStepRec), dens, sm);
}

// Kernel B: one 256-thread workgroup per (batch, head, 32 channels). Thread
// group g = tid / 32 owns the local and fine records j = g (mod 8);
// every record load is issued before any arithmetic and the groups merge in
// ascending g, so the summation order is fixed.
constexpr int kCombineCols = 32;
constexpr int kCombineGroups = kThreads / kCombineCols;
static_assert(kFineUnits % kCombineGroups == 0, "fine records split evenly over groups");

template <int D>
__global__ __launch_bounds__(kThreads) void decode_combine_kernel(DecodeParams p, int M) {
  using Gm = Geo<D>;
  constexpr int STRIDE = D + kStepRec, G = kCombineGroups, CHUNKS = D / kCombineCols;
  constexpr int NLOC = Gm::NLOC, LPG = (NLOC + G - 1) / G;
  __shared__ float ml[NLOC][2];
  __shared__ float part_num[G][kCombineCols], part_loc[G][kCombineCols];
  __shared__ float den_fine;
  const int bh = blockIdx.x / CHUNKS;
  const int chunk = blockIdx.x % CHUNKS;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, dc = tid % kCombineCols, g = tid / kCombineCols;
  const int d = chunk * kCombineCols + dc;
  const float* recs = p.parts + (size_t)bh * step_floats(D, p.sel_cap);
  const float* dens = recs + (NLOC + kFineUnits) * STRIDE;

  float m_g[LPG], l_g[LPG], o_g[LPG];
#pragma unroll
  for (int i = 0; i < LPG; ++i) {
    const int j = g + i * G;
    m_g[i] = j < NLOC ? recs[j * STRIDE] : -__builtin_inff();
    l_g[i] = j < NLOC ? recs[j * STRIDE + 1] : 0.0f;
    o_g[i] = j < NLOC ? recs[j * STRIDE + kStepRec + d] : 0.0f;
  }
  constexpr int FPG = kFineUnits / G;
  float n_v[FPG];
#pragma unroll
  for (int i = 0; i < FPG; ++i)
    n_v[i] = M > g + i * G ? recs[(NLOC + g + i * G) * STRIDE + kStepRec + d] : 0.0f;
  float q = 0.0f, a[3], bb[3];
  if (g == 0) {
    q = bf2f(p.rq.p[b * p.rq.sb + h * p.rq.sh + d]);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      a[i] = load_param(p.fa, p.f_dtype, h * p.fa_s[0] + d * p.fa_s[1] + i * p.fa_s[2]);
      bb[i] = load_param(p.fb, p.f_dtype, h * p.fb_s[0] + d * p.fb_s[1] + i * p.fb_s[2]);
    }
  }
  if (M > 0 && tid >= 64 && tid < 128) {
    // den = r(sum over slots of r(sum_d ch)), butterfly order over slots.
    const int lane = tid - 64;
    int slots = 64;
    while (slots < M) slots *= 2;
    const int per_lane = slots / 64;
    float vals[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int m = lane + 64 * k;
      vals[k] = (k < per_lane && m < M) ? dens[m] : 0.0f;
    }
    for (int width = per_lane; width > 1; width /= 2)
      for (int k = 0; k < width / 2; ++k) vals[k] += vals[k + width / 2];
    const float v = wave_sum_fold(vals[0]);
    if (lane == 0) den_fine = rbf(v);
  }
  if (dc == 0) {
#pragma unroll
    for (int i = 0; i < LPG; ++i)
      if (g + i * G < NLOC) { ml[g + i * G][0] = m_g[i]; ml[g + i * G][1] = l_g[i]; }
  }
  __syncthreads();
  float top = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < NLOC; ++j)
    if (ml[j][1] > 0.0f) top = fmaxf(top, ml[j][0]);
  float pl = 0.0f;
#pragma unroll
  for (int i = 0; i < LPG; ++i) pl += l_g[i] > 0.0f ? __expf(m_g[i] - top) * o_g[i] : 0.0f;
  float n_g = 0.0f;
#pragma unroll
  for (int i = 0; i < FPG; ++i) n_g += n_v[i];
  part_loc[g][dc] = pl;
  part_num[g][dc] = n_g;
  __syncthreads();
  if (g == 0) {
    float den_local = 0.0f;
#pragma unroll
    for (int j = 0; j < NLOC; ++j)
      if (ml[j][1] > 0.0f) den_local = fmaf(__expf(ml[j][0] - top), ml[j][1], den_local);
    float nl = 0.0f, nf = 0.0f;
#pragma unroll
    for (int gg = 0; gg < G; ++gg) { nl += part_loc[gg][dc]; nf += part_num[gg][dc]; }
    const float local = rbf(nl / den_local);
    bf16_t result;
    if (M > 0) {
      const float fine_v = rbf(rbf(nf) / den_fine);
      result = fuse_element(q, local, 0.0f, fine_v, a, bb, p.gain, 0, 1);
    } else {
      result = f2bf(local);
    }
    p.out[b * p.out_sb + h * p.out_sh + d] = result;
  }
  // Kernel A of this step has finished reading the position: advance it.
  if (blockIdx.x == 0 && tid == 0) p.header[0] = p.header[0] + 1;
}

__global__ __launch_bounds__(kThreads) void stage_tokens_kernel(StageParams p) {
  // One 16-byte chunk per thread: q, k, v, raw_q, raw_k rows of token 0.
  const int per_row = p.D / 8;
  const int bhn = p.B * p.H;
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= 5 * bhn * per_row) return;
  const int c = i % per_row, row = i / per_row;
  const int which = row / bhn, bh = row % bhn;
  const int b = bh / p.H, h = bh % p.H;
  TokView v;
  switch (which) {
    case 0: v = p.src[0]; break;
    case 1: v = p.src[1]; break;
    case 2: v = p.src[2]; break;
    case 3: v = p.src[3]; break;
    default: v = p.src[4]; break;
  }
  *(uint4*)(p.dst + ((size_t)which * bhn + bh) * p.D + c * 8) =
      *(const uint4*)(v.p + b * v.sb + h * v.sh + c * 8);
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

}  // namespace

hipError_t launch_decode_step(const DecodeParams& p, int head_dim, int M, hipStream_t s) {
  if (M < 0 || M > p.sel_cap || M > 512) return hipErrorInvalidValue;
  if (p.keep + p.fine > kMaxWindow) return hipErrorInvalidValue;
  const dim3 units((unsigned)(p.B * p.H * (local_units(head_dim) + kFineUnits)));
  const dim3 cols((unsigned)(p.B * p.H * (head_dim / kCombineCols)));
  if (head_dim == 128) {
    hipLaunchKernelGGL(decode_units_kernel<128>, units, dim3(kThreads), 0, s, p, M);
    hipLaunchKernelGGL(decode_combine_kernel<128>, cols, dim3(kThreads), 0, s, p, M);
  } else if (head_dim == 64) {
    hipLaunchKernelGGL(decode_units_kernel<64>, units, dim3(kThreads), 0, s, p, M);
    hipLaunchKernelGGL(decode_combine_kernel<64>, cols, dim3(kThreads), 0, s, p, M);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_stage_tokens(const StageParams& p, hipStream_t s) {
  const int chunks = 5 * p.B * p.H * (p.D / 8);
  hipLaunchKernelGGL(stage_tokens_kernel, dim3((unsigned)((chunks + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_ring_append(const AppendParams& p, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  hipLaunchKernelGGL(ring_append_kernel, dim3((unsigned)p.count, (unsigned)(p.B * p.H)),
                     dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace tao
