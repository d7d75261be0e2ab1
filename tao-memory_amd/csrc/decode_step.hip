// Fused single-token decode step for gfx950.
//
// Two launches per new token (replace, per request x layer, the reference's
// q1 page-memo region tao_stream.py:418-433 + query_fresh_fine.py:8-75, the
// local SDPA flash_attention.py:25-29 over torch.cat'ed K/V
// tao_stream.py:927-930, and the fusion kernels fusion_pointwise.py:10-117):
//
// decode_units_kernel: B*H*(kLocalSplits + M) independent workgroups
//   unit <  kLocalSplits : split-K exact local attention over the ring
//                          (split 0 also appends the new token to the ring)
//   unit >= kLocalSplits : one selected fine memory: streams its D x D bf16
//                          matrix from HBM (16-byte loads, 1 KB per wave
//                          instruction, all issued before any math; the
//                          bank stores C^T) and contracts it with the bf16
//                          channel weights ch = r(r(h*pw[page]) * sw[fine])
// decode_combine_kernel: one 1024-thread workgroup per (batch, head) merges the split-K
//   partials, sums the fine partials in a fixed order, den = r(sum_m r(sum_d
//   ch)) in butterfly order, fine = r(r(num)/den), applies the fusion
//   epilogue and advances header[0] (the stream position), so the pair can
//   be replayed from a hipGraph.
// The kernel boundary publishes the partials across the eight XCD L2
// caches; no device-scope fences or atomics are needed.
#include "tao_launch.h"
#include "tao_common.h"
#include "tao_fusion.h"

namespace tao {
namespace {

constexpr int kRec = 4;         // header floats per unit record
constexpr int kMaxLocal = 768;  // serve_limit: keys of one step's window

template <int D>
struct StepSmem {
  float vec[D];                         // query (local units) or ch (fine units)
  float red[kThreads / (D / 8) > D / 8 ? kThreads / (D / 8) : D / 8][D];  // partial sums
  float sc[64];                         // local scores of one split (<= 48)
  float misc[4];
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
__device__ void local_unit(const DecodeParams& p, int b, int h, int split,
                           long long position, int n_old, StepSmem<D>& sm,
                           float* rec) {
  constexpr int CH = D / 8, ROWS = kThreads / CH;
  constexpr int KPT = (kMaxLocal / kLocalSplits + ROWS - 1) / ROWS;   // keys per thread
  const int tid = threadIdx.x, c = tid % CH, r = tid / CH;
  const int L = p.keep + p.fine;
  const int n = n_old + 1;
  const int per = (n + kLocalSplits - 1) / kLocalSplits;
  const int j0 = min(n, split * per), j1 = min(n, j0 + per);
  const long long first_pos = position - n_old;
  const float scale = (float)(1.0 / __builtin_sqrt((double)D));

  const bf16_t* krow_new = p.k.p + b * p.k.sb + h * p.k.sh;
  const bf16_t* vrow_new = p.v.p + b * p.v.sb + h * p.v.sh;
  if (split == 0) {
    // Append the new token at slot position % L. No key of this step's
    // window occupies that slot (window length n_old <= L - 1).
    const int slot = (int)(position % L);
    const size_t off = (((size_t)b * L + slot) * p.H + h) * D;
    const bf16_t* rk = p.rk.p + b * p.rk.sb + h * p.rk.sh;
    for (int d = tid; d < D; d += kThreads) {
      p.ring_k[off + d] = krow_new[d];
      p.ring_v[off + d] = vrow_new[d];
      p.ring_raw[off + d] = rk[d];
    }
  }
  // Issue every load of this split first: q chunk, KPT key and value rows.
  uint4 kraw[KPT], vraw[KPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int j = j0 + r + i * ROWS;
    kraw[i] = make_uint4(0, 0, 0, 0);
    vraw[i] = make_uint4(0, 0, 0, 0);
    if (j < j1) {
      const bf16_t* krow;
      const bf16_t* vrow;
      if (j == n_old) {
        krow = krow_new;
        vrow = vrow_new;
      } else {
        const size_t off = (((size_t)b * L + (int)((first_pos + j) % L)) * p.H + h) * D;
        krow = p.ring_k + off;
        vrow = p.ring_v + off;
      }
      kraw[i] = *(const uint4*)(krow + c * 8);
      vraw[i] = *(const uint4*)(vrow + c * 8);
    }
  }
  float qv[8];
  unpack8(*(const uint4*)(p.q.p + b * p.q.sb + h * p.q.sh + c * 8), qv);
  float score[KPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    float kv[8];
    unpack8(kraw[i], kv);
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) part = fmaf(qv[e], kv[e], part);
    score[i] = group_sum<CH>(part) * scale;
    const int j = j0 + r + i * ROWS;
    if (j < j1 && c == 0) sm.sc[j - j0] = score[i];
  }
  __syncthreads();
  const int cnt = j1 - j0;
  if (tid < 64) {
    const float a = tid < cnt ? sm.sc[tid] : -__builtin_inff();
    const float top = wave_max(a);
    const float e = wave_sum_fold(tid < cnt ? __expf(a - top) : 0.0f);
    if (tid == 0) { sm.misc[0] = top; sm.misc[1] = e; }
  }
  __syncthreads();
  const float top = sm.misc[0];
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int j = j0 + r + i * ROWS;
    if (j < j1) {
      const float w = __expf(score[i] - top);
      float vv[8];
      unpack8(vraw[i], vv);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(w, vv[e], acc[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) sm.red[r][c * 8 + e] = acc[e];
  __syncthreads();
  if (tid < D) {
    float s = 0.0f;
    for (int rr = 0; rr < ROWS; ++rr) s += sm.red[rr][tid];
    rec[kRec + tid] = s;
  }
  if (tid == 0) {
    rec[0] = cnt > 0 ? top : -__builtin_inff();
    rec[1] = cnt > 0 ? sm.misc[1] : 0.0f;
  }
}

template <int D>
__device__ void fine_unit(const DecodeParams& p, int b, int h, int m,
                          StepSmem<D>& sm, float* rec) {
  constexpr int CH = D / 8, ROWS = kThreads / CH, RPT = D / ROWS, PER = D / 64;
  const int tid = threadIdx.x, c = tid % CH, r = tid / CH;
  const int bh = b * p.H + h;
  const int id = p.sel[(size_t)bh * p.sel_cap + m];
  const int page = id / p.group;
  const bf16_t* cmat = p.bank + ((size_t)bh * p.fine_cap + id) * D * D;

  // Issue the whole matrix stream first; h / ch are computed under it.
  uint4 cv[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    cv[i] = *(const uint4*)(cmat + (size_t)(r + i * ROWS) * D + c * 8);

  if (tid < 64) {
    const bf16_t* rq = p.rq.p + b * p.rq.sb + h * p.rq.sh;
    const bf16_t* pw = p.pw + ((size_t)bh * p.page_cap + page) * D;
    const bf16_t* sw = p.sw + ((size_t)bh * p.fine_cap + id) * D;
    float x[PER], pwv[PER], swv[PER], e[PER];
    float top = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      x[k] = bf2f(rq[tid + 64 * k]);
      pwv[k] = bf2f(pw[tid + 64 * k]);
      swv[k] = bf2f(sw[tid + 64 * k]);
      top = fmaxf(top, x[k]);
    }
    top = wave_max(top);
#pragma unroll
    for (int k = 0; k < PER; ++k) e[k] = exp_cr(x[k] - top);
    float s = e[0];
#pragma unroll
    for (int k = 1; k < PER; ++k) s += e[k];   // PER <= 2: fold of the lane pair
    s = wave_sum_fold(s);
    float csum = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int d = tid + 64 * k;
      const float hq = rbf(e[k] / s);
      const float hv = rbf(hq * pwv[k]);
      const float ch = rbf(hv * swv[k]);
      sm.vec[d] = ch;
      csum = k == 0 ? ch : csum + ch;
    }
    csum = wave_sum_fold(csum);
    if (tid == 0) sm.misc[0] = rbf(csum);
  }
  __syncthreads();
  // Bank rows are C^T[e][d]: this thread holds d in [8c, 8c + 8) of rows
  // e = r + i * ROWS; partial dots are summed over the CH chunks in LDS.
  float chv[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) chv[k] = sm.vec[c * 8 + k];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    float cf[8];
    unpack8(cv[i], cf);
    float part = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) part = fmaf(chv[k], cf[k], part);
    sm.red[c][r + i * ROWS] = part;
  }
  __syncthreads();
  if (tid < D) {
    float s = 0.0f;
    for (int cc = 0; cc < CH; ++cc) s += sm.red[cc][tid];
    rec[kRec + tid] = s;
  }
  if (tid == 0) rec[0] = sm.misc[0];
}

// Kernel A: independent units, no cross-workgroup communication.
template <int D>
__global__ __launch_bounds__(kThreads) void decode_units_kernel(DecodeParams p, int M) {
  __shared__ StepSmem<D> sm;
  const int units = kLocalSplits + M;
  const int bh = blockIdx.x / units;
  const int unit = blockIdx.x % units;
  const int b = bh / p.H, h = bh % p.H;
  float* recs = p.parts + (size_t)bh * (kLocalSplits + p.sel_cap) * (D + kRec);
  if (unit < kLocalSplits) {
    const long long position = p.header[0];
    const int n_old = local_len_at(position, p.keep, p.fine);
    local_unit<D>(p, b, h, unit, position, n_old, sm, recs + unit * (D + kRec));
  } else {
    fine_unit<D>(p, b, h, unit - kLocalSplits, sm, recs + unit * (D + kRec));
  }
}

// Kernel B: one 1024-thread workgroup per (batch, head). Thread group
// g = tid / D owns local splits s = g (mod G) and fine slots m = g (mod G);
// every record load is issued before any arithmetic, and the groups merge in
// ascending g, so the summation order is fixed.
constexpr int kCombineThreads = 1024;

template <int D>
__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(DecodeParams p, int M) {
  constexpr int STRIDE = D + kRec, G = kCombineThreads / D;
  constexpr int SPG = kLocalSplits / G > 0 ? kLocalSplits / G : 1;   // splits per group
  constexpr int UNROLL = 8;
  __shared__ float ml[kLocalSplits][2];
  __shared__ float part_num[G][D], part_loc[G][D];
  __shared__ float den_local, den_fine;
  const int bh = blockIdx.x;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, d = tid % D, g = tid / D;
  const float* recs = p.parts + (size_t)bh * (kLocalSplits + p.sel_cap) * STRIDE;

  if (tid < 2 * kLocalSplits) ml[tid >> 1][tid & 1] = recs[(tid >> 1) * STRIDE + (tid & 1)];
  float accl[SPG];
#pragma unroll
  for (int i = 0; i < SPG; ++i) {
    const int s = g + i * G;
    accl[i] = s < kLocalSplits ? recs[s * STRIDE + kRec + d] : 0.0f;
  }
  float num_f = 0.0f;
  const float* fine = recs + (size_t)kLocalSplits * STRIDE + kRec + d;
  for (int base = g; base < M; base += UNROLL * G) {
    float v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int m = base + u * G;
      v[u] = m < M ? fine[(size_t)m * STRIDE] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) num_f = num_f + v[u];
  }
  if (M > 0 && tid < 64) {
    // den = r(sum over slots of r(sum_d ch)), butterfly order over slots.
    int slots = 64;
    while (slots < M) slots *= 2;
    const int per_lane = slots / 64;
    float vals[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int m = tid + 64 * k;
      vals[k] = (k < per_lane && m < M) ? recs[(kLocalSplits + m) * STRIDE] : 0.0f;
    }
    for (int width = per_lane; width > 1; width /= 2)
      for (int k = 0; k < width / 2; ++k) vals[k] += vals[k + width / 2];
    const float v = wave_sum_fold(vals[0]);
    if (tid == 0) den_fine = rbf(v);
  }
  __syncthreads();
  float top = -__builtin_inff();
#pragma unroll
  for (int s = 0; s < kLocalSplits; ++s)
    if (ml[s][1] > 0.0f) top = fmaxf(top, ml[s][0]);
  float num_l = 0.0f;
#pragma unroll
  for (int i = 0; i < SPG; ++i) {
    const int s = g + i * G;
    if (s < kLocalSplits && ml[s][1] > 0.0f) num_l = fmaf(__expf(ml[s][0] - top), accl[i], num_l);
  }
  part_loc[g][d] = num_l;
  part_num[g][d] = num_f;
  if (tid == 0) {
    float den = 0.0f;
#pragma unroll
    for (int s = 0; s < kLocalSplits; ++s)
      if (ml[s][1] > 0.0f) den = fmaf(__expf(ml[s][0] - top), ml[s][1], den);
    den_local = den;
  }
  __syncthreads();
  if (tid < D) {
    float nl = 0.0f, nf = 0.0f;
#pragma unroll
    for (int gg = 0; gg < G; ++gg) { nl += part_loc[gg][d]; nf += part_num[gg][d]; }
    const float local = rbf(nl / den_local);
    bf16_t result;
    if (M > 0) {
      const float fine_v = rbf(rbf(nf) / den_fine);
      const float q = bf2f(p.rq.p[b * p.rq.sb + h * p.rq.sh + d]);
      float a[3], bb[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        a[i] = load_param(p.fa, p.f_dtype, h * p.fa_s[0] + d * p.fa_s[1] + i * p.fa_s[2]);
        bb[i] = load_param(p.fb, p.f_dtype, h * p.fb_s[0] + d * p.fb_s[1] + i * p.fb_s[2]);
      }
      result = fuse_element(q, local, 0.0f, fine_v, a, bb, p.gain, 0, 1);
    } else {
      result = f2bf(local);
    }
    p.out[b * p.out_sb + h * p.out_sh + d] = result;
  }
  // Kernel A of this step has finished reading the position: advance it.
  if (bh == 0 && tid == 0) p.header[0] = p.header[0] + 1;
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
  const dim3 units((unsigned)(p.B * p.H * (kLocalSplits + M)));
  const dim3 heads((unsigned)(p.B * p.H));
  if (head_dim == 128) {
    hipLaunchKernelGGL(decode_units_kernel<128>, units, dim3(kThreads), 0, s, p, M);
    hipLaunchKernelGGL(decode_combine_kernel<128>, heads, dim3(kCombineThreads), 0, s, p, M);
  } else if (head_dim == 64) {
    hipLaunchKernelGGL(decode_units_kernel<64>, units, dim3(kThreads), 0, s, p, M);
    hipLaunchKernelGGL(decode_combine_kernel<64>, heads, dim3(kCombineThreads), 0, s, p, M);
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
