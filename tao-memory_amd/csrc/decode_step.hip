// Fused single-token decode step for gfx950.
//
// One launch per new token (replaces, per request x layer, the reference's
// q1 page-memo region tao_stream.py:418-433 + query_fresh_fine.py:8-75, the
// local SDPA flash_attention.py:25-29 over torch.cat'ed K/V
// tao_stream.py:927-930, and the fusion kernels fusion_pointwise.py:10-117):
//
//   grid = B*H*(kLocalSplits + M) workgroups of 256 threads
//   unit <  kLocalSplits : split-K exact local attention over the ring
//                          (split 0 also appends the new token to the ring)
//   unit >= kLocalSplits : one selected fine memory: streams its D x D bf16
//                          matrix from HBM (16-byte loads, 1 KB per wave
//                          instruction) and contracts it with the bf16
//                          channel weights ch = r(r(h*pw[page]) * sw[fine])
//   last arriving unit of a head: merges the split-K partials, sums the M
//   fine partials in slot order (deterministic), den = r(sum_m r(sum_d ch)),
//   fine = r(r(num)/den), then the fusion epilogue writes the output row.
//   The last head to finish advances header[0] (the stream position), so the
//   same launch can be replayed from a hipGraph.
#include "tao_launch.h"
#include "tao_common.h"
#include "tao_fusion.h"

namespace tao {
namespace {

constexpr int kRec = 4;   // header floats per unit record

template <int D>
struct StepSmem {
  float vec[D];                         // query (local units) or ch (fine units)
  float red[kThreads / (D / 8)][D];     // cross-row partial sums
  float sc[128];                        // local scores of one split (<= 96)
  float misc[4];
  int last;
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

  float qv[8];
  {
    const bf16_t* qrow = p.q.p + b * p.q.sb + h * p.q.sh;
    unpack8(*(const uint4*)(qrow + c * 8), qv);
  }
  for (int base = j0; base < j1; base += ROWS) {
    const int j = base + r;
    const bool valid = j < j1;
    float part = 0.0f;
    if (valid) {
      const bf16_t* krow;
      if (j == n_old) {
        krow = krow_new;
      } else {
        const int slot = (int)((first_pos + j) % L);
        krow = p.ring_k + (((size_t)b * L + slot) * p.H + h) * D;
      }
      float kv[8];
      unpack8(*(const uint4*)(krow + c * 8), kv);
#pragma unroll
      for (int i = 0; i < 8; ++i) part = fmaf(qv[i], kv[i], part);
    }
    part = group_sum<CH>(part);
    if (valid && c == 0) sm.sc[j - j0] = part * scale;
  }
  __syncthreads();
  const int cnt = j1 - j0;
  if (tid < 64) {
    float a = tid < cnt ? sm.sc[tid] : -__builtin_inff();
    float bb = tid + 64 < cnt ? sm.sc[tid + 64] : -__builtin_inff();
    float top = wave_max(fmaxf(a, bb));
    float e = (tid < cnt ? __expf(a - top) : 0.0f) + (tid + 64 < cnt ? __expf(bb - top) : 0.0f);
    e = wave_sum_fold(e);
    if (tid == 0) { sm.misc[0] = top; sm.misc[1] = e; }
  }
  __syncthreads();
  const float top = sm.misc[0];
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int j = j0 + r; j < j1; j += ROWS) {
    const float w = __expf(sm.sc[j - j0] - top);
    const bf16_t* vrow;
    if (j == n_old) {
      vrow = vrow_new;
    } else {
      const int slot = (int)((first_pos + j) % L);
      vrow = p.ring_v + (((size_t)b * L + slot) * p.H + h) * D;
    }
    float vv[8];
    unpack8(*(const uint4*)(vrow + c * 8), vv);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = fmaf(w, vv[i], acc[i]);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) sm.red[r][c * 8 + i] = acc[i];
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
    float x[PER], e[PER];
    float top = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < PER; ++k) { x[k] = bf2f(rq[tid + 64 * k]); top = fmaxf(top, x[k]); }
    top = wave_max(top);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) e[k] = exp_cr(x[k] - top);
    s = e[0];
#pragma unroll
    for (int k = 1; k < PER; ++k) s += e[k];   // PER <= 2: fold of the lane pair
    s = wave_sum_fold(s);
    float csum = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int d = tid + 64 * k;
      const float hq = rbf(e[k] / s);
      const float hv = rbf(hq * bf2f(pw[d]));
      const float ch = rbf(hv * bf2f(sw[d]));
      sm.vec[d] = ch;
      csum = k == 0 ? ch : csum + ch;
    }
    csum = wave_sum_fold(csum);
    if (tid == 0) sm.misc[0] = rbf(csum);
  }
  __syncthreads();
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const float w = sm.vec[r + i * ROWS];
    float cf[8];
    unpack8(cv[i], cf);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = fmaf(w, cf[k], acc[k]);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) sm.red[r][c * 8 + k] = acc[k];
  __syncthreads();
  if (tid < D) {
    float s = 0.0f;
    for (int rr = 0; rr < ROWS; ++rr) s += sm.red[rr][tid];
    rec[kRec + tid] = s;
  }
  if (tid == 0) rec[0] = sm.misc[0];
}

template <int D>
__device__ void combine(const DecodeParams& p, int b, int h, int M,
                        StepSmem<D>& sm, const float* recs) {
  constexpr int STRIDE = D + kRec;
  const int tid = threadIdx.x;
  if (M > 0 && tid < 64) {
    // den = r(sum over slots of r(sum_d ch)), butterfly order over slots.
    float v = 0.0f;
    int slots = 64;
    while (slots < M) slots *= 2;
    float vals[8];
    const int per_lane = slots / 64;
    for (int k = 0; k < per_lane && k < 8; ++k) {
      const int m = tid + 64 * k;
      vals[k] = m < M ? recs[(kLocalSplits + m) * STRIDE] : 0.0f;
    }
    for (int width = per_lane; width > 1; width /= 2)
      for (int k = 0; k < width / 2; ++k) vals[k] += vals[k + width / 2];
    v = wave_sum_fold(vals[0]);
    if (tid == 0) sm.misc[2] = rbf(v);
  }
  __syncthreads();
  if (tid < D) {
    float top = -__builtin_inff();
    for (int s = 0; s < kLocalSplits; ++s) {
      const float* rs = recs + s * STRIDE;
      if (rs[1] > 0.0f) top = fmaxf(top, rs[0]);
    }
    float num = 0.0f, den = 0.0f;
    for (int s = 0; s < kLocalSplits; ++s) {
      const float* rs = recs + s * STRIDE;
      if (rs[1] > 0.0f) {
        const float w = __expf(rs[0] - top);
        den = fmaf(w, rs[1], den);
        num = fmaf(w, rs[kRec + tid], num);
      }
    }
    const float local = rbf(num / den);
    bf16_t result;
    if (M > 0) {
      float acc = 0.0f;
      for (int m = 0; m < M; ++m) acc += recs[(kLocalSplits + m) * STRIDE + kRec + tid];
      const float fine = rbf(rbf(acc) / sm.misc[2]);
      const float q = bf2f(p.rq.p[b * p.rq.sb + h * p.rq.sh + tid]);
      float a[3], bb[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        a[i] = load_param(p.fa, p.f_dtype, h * p.fa_s[0] + tid * p.fa_s[1] + i * p.fa_s[2]);
        bb[i] = load_param(p.fb, p.f_dtype, h * p.fb_s[0] + tid * p.fb_s[1] + i * p.fb_s[2]);
      }
      result = fuse_element(q, local, 0.0f, fine, a, bb, p.gain, 0, 1);
    } else {
      result = f2bf(local);
    }
    p.out[b * p.out_sb + h * p.out_sh + tid] = result;
  }
}

template <int D>
__global__ __launch_bounds__(kThreads) void decode_step_kernel(DecodeParams p, int M) {
  __shared__ StepSmem<D> sm;
  const int units = kLocalSplits + M;
  const int bh = blockIdx.x / units;
  const int unit = blockIdx.x % units;
  const int b = bh / p.H, h = bh % p.H;
  float* recs = p.parts + (size_t)bh * (kLocalSplits + p.sel_cap) * (D + kRec);
  const long long position = p.header[0];
  if (unit < kLocalSplits) {
    const int n_old = local_len_at(position, p.keep, p.fine);
    local_unit<D>(p, b, h, unit, position, n_old, sm, recs + unit * (D + kRec));
  } else {
    fine_unit<D>(p, b, h, unit - kLocalSplits, sm, recs + unit * (D + kRec));
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = atomicAdd(&p.counters[bh], 1u);
    sm.last = prev == (unsigned)(units - 1);
  }
  __syncthreads();
  if (!sm.last) return;
  __threadfence();
  combine<D>(p, b, h, M, sm, recs);
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    atomicExch(&p.counters[bh], 0u);
    const unsigned total = (unsigned)(p.B * p.H);
    const unsigned prev = atomicAdd(&p.counters[total], 1u);
    if (prev == total - 1) {
      atomicExch(&p.counters[total], 0u);
      atomicAdd((unsigned long long*)&p.header[0], 1ull);
    }
  }
}

__global__ __launch_bounds__(kThreads) void stage_tokens_kernel(StageParams p) {
  // One workgroup per (b, h): copies q, k, v, raw_q, raw_k rows (token 0).
  const int bh = blockIdx.x;
  const int b = bh / p.H, h = bh % p.H;
  for (int i = threadIdx.x; i < 5 * p.D; i += kThreads) {
    const int which = i / p.D, d = i % p.D;
    const TokView& v = p.src[which];
    p.dst[((size_t)which * p.B * p.H + bh) * p.D + d] = v.p[b * v.sb + h * v.sh + d];
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

}  // namespace

hipError_t launch_decode_step(const DecodeParams& p, int head_dim, int M, hipStream_t s) {
  const dim3 grid((unsigned)(p.B * p.H * (kLocalSplits + M)));
  if (head_dim == 128)
    hipLaunchKernelGGL(decode_step_kernel<128>, grid, dim3(kThreads), 0, s, p, M);
  else if (head_dim == 64)
    hipLaunchKernelGGL(decode_step_kernel<64>, grid, dim3(kThreads), 0, s, p, M);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_stage_tokens(const StageParams& p, hipStream_t s) {
  hipLaunchKernelGGL(stage_tokens_kernel, dim3((unsigned)(p.B * p.H)), dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_ring_append(const AppendParams& p, hipStream_t s) {
  if (p.count <= 0) return hipSuccess;
  hipLaunchKernelGGL(ring_append_kernel, dim3((unsigned)p.count, (unsigned)(p.B * p.H)),
                     dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace tao
