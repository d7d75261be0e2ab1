// fp32 full-sequence read: tao_attention on fp32 operands.
//
// Reference: tao_attention (operator.py:40-54) = read_training
// (tao_stream.py:668-757, route_interval=1) followed by _fuse_training
// (operator.py:21-38), with the softmax fine writer of _seal_training_all
// (tao_stream.py:80-123), the page metadata of _training_metadata /
// _tile_metadata (:530-593), the local tiles of _local_training_corrected_4k
// (:760-787) and the per-query route and read of _read_training_group
// (:596-665).
//
// fp32 semantics. The reference's torch operations follow the operand dtype;
// its Triton kernels hard-cast their products to bf16 (routing_scores.py:28,
// selected_read.py:31, 48), which has no fp32 meaning. Here every rounding
// point of the bf16 contract rounds to fp32 instead, so:
//  * everything that decides a route is bit-reproducible: exp and log are
//    fp64 evaluations rounded once to fp32; sums over channels, pages and
//    slots use the butterfly order (pad to a power of two, add the upper half
//    onto the lower); the writer's token sums run four sequential 64-token
//    quarters added pairwise; every product and sum is one IEEE fp32
//    operation (no contraction in this file);
//  * the local attention, the value matrices, the coarse read and the
//    selected read's numerator accumulate in fp32 in their own order, within
//    the 1e-4 tolerance of exact arithmetic.
// These kernels are VALU code: the fp32 path serves parity at the reference's
// CPU-eager configuration, not throughput.
#pragma clang fp contract(off)

#include "schedule.h"
#include "tao_common.h"
#include "tao_fusion.h"
#include "tao_launch.h"

namespace tao {
namespace {

constexpr int kFine = 256;          // fine_tokens
constexpr int kGroup = 8;           // coarse_group
constexpr int kKeep = 512;          // local_keep
constexpr int kRowsPerPage = 36;    // segment-weight rows of a page: prefixes n = 1..8
constexpr int kChunk = 16;          // queries per read block
constexpr int kKeyStage = 16;       // keys per local-attention LDS stage
constexpr int kVChunk = 32;         // value rows per writer LDS stage
constexpr float kLogTwoF32 = 0.693147180559945309f;   // fp32(log 2)

TAO_DEV float ld(const F32View& v, int b, int64_t t, int h, int d) {
  return v.p[b * v.sb + t * v.st + h * v.sh + d];
}

TAO_DEV float wave_max(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}

// Butterfly sum of the 64 lanes' values (fold halves: lane i adds lane
// i + half for half = 32 .. 1), broadcast to every lane.
TAO_DEV float wave_fold(float x) {
#pragma unroll
  for (int half = 32; half >= 1; half >>= 1) x = x + __shfl_down(x, half);
  return __shfl(x, 0);
}

// Butterfly sum over the D channels held as lane + 64 r (R = D / 64).
template <int R>
TAO_DEV float channel_fold(const float (&x)[R]) {
  float s = x[0];
  if constexpr (R == 2) s = x[0] + x[1];
  return wave_fold(s);
}

// Butterfly sum of n values held as lane + 64 k (k < K slots, n <= 64 K).
template <int K>
TAO_DEV float slot_fold(float (&x)[K], int n) {
  int width = 1;
  while (width < n) width <<= 1;
  const int lane = threadIdx.x & 63;
  float v[K];
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = (lane + 64 * k) < n ? x[k] : 0.0f;
  for (int half = width / 2; half >= 64; half >>= 1) {
    const int step = half / 64;
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (k < step) v[k] = v[k] + v[k + step < K ? k + step : k];
  }
  return wave_fold(v[0]);
}

// --------------------------------------------------------------- local tiles
// Query t of tile j attends causally to keys [max(0, 256 j - 512), t]
// (_local_training_corrected_4k and its ragged fallback); softmax scale
// 1/sqrt(D) as SDPA's default. A workgroup takes 64 queries (lane t0 + i of
// every wave holds query t0 + i) and splits their key range by 16-key stages
// over its kLocalWaves(D) waves (stage s to wave s % waves), each wave with
// its own LDS stage and online softmax (m, l, acc); the waves' partials are
// merged in wave order: M = max m_w, l = sum l_w e^(m_w - M),
// o = sum acc_w e^(m_w - M) / l.
template <int D> constexpr int kLocalWaves = D == 64 ? 8 : 4;
constexpr int kMergeCols = 16;       // channels per merge round

template <int D>
__global__ __launch_bounds__(64 * kLocalWaves<D>) void f32_local_kernel(F32Params p) {
  constexpr int NW = kLocalWaves<D>;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int h = blockIdx.y, b = blockIdx.z;
  const int t0 = blockIdx.x * 64;
  const int t = t0 + lane;
  const bool active = t < p.T;
  const int k0 = max(0, (t0 / kFine) * kFine - kKeep);
  const int k1 = min(p.T, t0 + 64);
  __shared__ float ks[NW][kKeyStage][D], vs[NW][kKeyStage][D];
  __shared__ float wm[NW][64], wl[NW][64];
  const float scale = 1.0f / sqrtf((float)D);
  float q[D], acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    q[d] = active ? ld(p.q, b, t, h, d) : 0.0f;
    acc[d] = 0.0f;
  }
  float m = -__builtin_inff(), l = 0.0f;
  for (int kb = k0 + w * kKeyStage; kb < k1; kb += NW * kKeyStage) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int i = lane; i < kKeyStage * D; i += 64) {
      const int j = i / D, d = i % D, key = kb + j;
      ks[w][j][d] = key < k1 ? ld(p.k, b, key, h, d) : 0.0f;
      vs[w][j][d] = key < k1 ? ld(p.v, b, key, h, d) : 0.0f;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float s[kKeyStage];
    float cm = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < kKeyStage; ++j) {
      s[j] = -__builtin_inff();
      if (active && kb + j <= t) {
        float dot = 0.0f;
#pragma unroll
        for (int d = 0; d < D; ++d) dot = fmaf(q[d], ks[w][j][d], dot);
        s[j] = dot * scale;
        cm = fmaxf(cm, s[j]);
      }
    }
    if (cm > -__builtin_inff()) {
      const float mn = fmaxf(m, cm);
      const float corr = expf(m - mn);
      l *= corr;
#pragma unroll
      for (int d = 0; d < D; ++d) acc[d] *= corr;
#pragma unroll
      for (int j = 0; j < kKeyStage; ++j) {
        const float wgt = expf(s[j] - mn);
        l += wgt;
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = fmaf(wgt, vs[w][j][d], acc[d]);
      }
      m = mn;
    }
  }
  // Merge the waves' partials (a wave with no key of a query has m = -inf
  // and weighs 0; every query sees its own key, so M is finite).
  wm[w][lane] = m;
  wl[w][lane] = l;
  __syncthreads();
  float top = wm[0][lane];
#pragma unroll
  for (int v = 1; v < NW; ++v) top = fmaxf(top, wm[v][lane]);
  const float f = m > -__builtin_inff() ? expf(m - top) : 0.0f;
  float lsum = 0.0f;
#pragma unroll
  for (int v = 0; v < NW; ++v)
    lsum += wm[v][lane] > -__builtin_inff() ? wl[v][lane] * expf(wm[v][lane] - top) : 0.0f;
  // Channel rounds through the (now free) key stages: wave w's scaled
  // partials of kMergeCols channels, then lane i of wave w sums query i's
  // channels w, w + NW, ... of the round over the waves in order.
  float* red = &ks[0][0][0];                       // [NW][64][kMergeCols]
  static_assert(NW * 64 * kMergeCols <= NW * kKeyStage * D, "merge buffer fits the stages");
  float* o = p.local + (((size_t)b * p.T + (active ? t : 0)) * p.H + h) * D;
#pragma unroll
  for (int c0 = 0; c0 < D; c0 += kMergeCols) {
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kMergeCols; ++c) red[(w * 64 + lane) * kMergeCols + c] = acc[c0 + c] * f;
    __syncthreads();
    for (int c = w; c < kMergeCols; c += NW) {
      float sum = 0.0f;
#pragma unroll
      for (int v = 0; v < NW; ++v) sum += red[(v * 64 + lane) * kMergeCols + c];
      if (active) o[c0 + c] = sum / lsum;
    }
  }
}

// ------------------------------------------------------------------- writer
// One visible block (fine f) of one head: per channel d over its 256 tokens,
// top = max k, e = exp(k - top), Z = quarter sums, P = e / Z,
// z = top + log Z; then C[d][e] = sum_t P[t][d] v[t][e].
template <int D>
__global__ __launch_bounds__(4 * D) void f32_writer_kernel(F32Params p) {
  const int f = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int d = tid % D, quarter = tid / D;
  __shared__ float prob[kFine][D];
  __shared__ float red[4][D];
  __shared__ float vchunk[kVChunk][D];
  const int64_t base = (int64_t)f * kFine;
  float top = -__builtin_inff();
  for (int i = 0; i < 64; ++i) top = fmaxf(top, ld(p.rk, b, base + quarter * 64 + i, h, d));
  red[quarter][d] = top;
  __syncthreads();
  top = fmaxf(fmaxf(red[0][d], red[1][d]), fmaxf(red[2][d], red[3][d]));
  __syncthreads();
  float acc = 0.0f;
  for (int i = 0; i < 64; ++i) {
    const int tok = quarter * 64 + i;
    const float e = exp_cr(ld(p.rk, b, base + tok, h, d) - top);
    prob[tok][d] = e;
    acc = acc + e;
  }
  red[quarter][d] = acc;
  __syncthreads();
  const float total = (red[0][d] + red[1][d]) + (red[2][d] + red[3][d]);
  for (int i = 0; i < 64; ++i) {
    const int tok = quarter * 64 + i;
    prob[tok][d] = prob[tok][d] / total;
  }
  const size_t bh = (size_t)b * p.H + h;
  if (quarter == 0) p.fine_z[(bh * p.S + f) * D + d] = top + log_cr(total);
  __syncthreads();
  constexpr int E = D / 4;
  const int row = tid / 4, part = tid % 4;
  float c[E];
#pragma unroll
  for (int e = 0; e < E; ++e) c[e] = 0.0f;
  // v staged kVChunk tokens at a time (the token order of the sums is kept).
  for (int c0 = 0; c0 < kFine; c0 += kVChunk) {
    __syncthreads();
    for (int i = tid; i < kVChunk * D; i += 4 * D) {
      const int tt = i / D, e = i % D;
      vchunk[tt][e] = ld(p.v, b, base + c0 + tt, h, e);
    }
    __syncthreads();
    for (int tt = 0; tt < kVChunk; ++tt) {
      const float pr = prob[c0 + tt][row];
#pragma unroll
      for (int e = 0; e < E; ++e) c[e] = fmaf(pr, vchunk[tt][part * E + e], c[e]);
    }
  }
  float* out = p.bank + ((bh * p.S + f) * D + row) * D + part * E;
#pragma unroll
  for (int e = 0; e < E; ++e) out[e] = c[e];
}

// -------------------------------------------------------------------- pages
// Page pg: pz[n - 1] = logsumexp of its first n fines for every prefix n
// present (a completed page's summary is n = 8, a pending page's the prefix
// a tile sees), the segment weights exp(z - pz[n - 1]) of those n fines, and,
// with coarse values, the completed page's value matrix
// PC[d][e] = sum_s w_s[d] C_s[d][e] (tao_stream.py:486-499).
template <int D>
__global__ __launch_bounds__(D) void f32_pages_kernel(F32Params p) {
  const int pg = blockIdx.x, h = blockIdx.y, b = blockIdx.z, d = threadIdx.x;
  const size_t bh = (size_t)b * p.H + h;
  const int first = pg * kGroup;
  const int avail = min(kGroup, p.S - first);
  float z[kGroup];
#pragma unroll
  for (int i = 0; i < kGroup; ++i) z[i] = i < avail ? p.fine_z[(bh * p.S + first + i) * D + d] : 0.0f;
  float* pz = p.pz + (bh * p.P8 + pg) * kGroup * D;
  float* sw = p.swt + (bh * p.P8 + pg) * kRowsPerPage * D;
  float wfull[kGroup];
  for (int n = 1; n <= avail; ++n) {
    float top = -__builtin_inff();
    for (int i = 0; i < n; ++i) top = fmaxf(top, z[i]);
    if (__builtin_isinf(top)) top = 0.0f;
    float e[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; ++i) e[i] = i < n ? exp_cr(z[i] - top) : 0.0f;
    int width = 1;
    while (width < n) width <<= 1;
    for (int half = width / 2; half >= 1; half >>= 1)
#pragma unroll
      for (int i = 0; i < kGroup / 2; ++i)
        if (i < half) e[i] = e[i] + e[i + half];
    const float v = log_cr(e[0]) + top;
    pz[(n - 1) * D + d] = v;
    const int row0 = n * (n - 1) / 2;
    for (int j = 0; j < n; ++j) {
      const float w = exp_cr(z[j] - v);
      sw[(row0 + j) * D + d] = w;
      if (n == kGroup) wfull[j] = w;
    }
  }
  if (p.pc && avail == kGroup) {
    const float* c = p.bank + ((bh * p.S + first) * D + d) * D;
    float* out = p.pc + ((bh * p.Pc + pg) * D + d) * D;
    for (int e = 0; e < D; ++e) {
      float acc = 0.0f;
#pragma unroll
      for (int s = 0; s < kGroup; ++s) acc = fmaf(wfull[s], c[(size_t)s * D * D + e], acc);
      out[e] = acc;
    }
  }
}

// --------------------------------------------------------------------- read
// kChunk queries of one tile and head per block (one wave). Tile prologue:
// the pages the tile sees (completed pages' summaries, the pending page's
// prefix summary), page weights softmax over them per channel and, with
// coarse values, the coarse weights softmax over the completed pages. Per
// query: h = softmax(raw_q), hv = h * pw, page masses, the chosen pages,
// candidate masses, the stable top-M, the selected read, the coarse read and
// the fusion.
constexpr int kMaxPages = 64;
constexpr int kMaxCand = 256;
constexpr int kReadWaves = 4;        // waves per block; wave w reads queries t0 + w + 4 k

// Orders one wave's LDS accesses across its lanes (scratch private to a wave).
TAO_DEV void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

TAO_DEV int stable_rank(float mine, int idx, int n, const float* all) {
  int r = 0;
  for (int j = 0; j < n; ++j) {
    const float o = all[j];
    r += (o > mine) || (o == mine && j < idx);
  }
  return r;
}

template <int D>
__global__ __launch_bounds__(64 * kReadWaves) void f32_read_kernel(F32Params p) {
  constexpr int R = D / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int h = blockIdx.y, b = blockIdx.z;
  const int t0 = blockIdx.x * kChunk;
  const int tend = min(p.T, t0 + kChunk);
  const int tile = t0 / kFine;
  const int visible = max(0, tile - kKeep / kFine);
  const size_t bh = (size_t)b * p.H + h;
  auto out_at = [&](int t, int d) -> float* {
    return p.out + b * p.out_sb + (int64_t)t * p.out_st + h * p.out_sh + d;
  };
  const float* local = p.local;
  if (!visible) {   // neither history branch present: the output is local
    for (int t = t0 + w; t < tend; t += kReadWaves) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        *out_at(t, lane + 64 * r) = local[(((size_t)b * p.T + t) * p.H + h) * D + lane + 64 * r];
      if (p.sel_out)
        for (int m = lane; m < p.sel_cap; m += 64)
          p.sel_out[(((size_t)b * p.T + t) * p.H + h) * p.sel_cap + m] = -1;
    }
    return;
  }
  const int completed = visible / kGroup, pending = visible % kGroup;
  const int P = completed + (pending > 0);
  int64_t coarse64 = 0, elig64 = 0, sel64 = 0;
  sched::routed_counts(p.cfg, completed, pending, &coarse64, &elig64, &sel64);
  const int coarse = (int)coarse64, M = (int)sel64;
  const bool coarse_on = p.coarse_values && tile * kFine >= kKeep + kGroup * kFine;

  __shared__ float pw[kMaxPages][D];
  __shared__ float cw[kMaxPages][D];
  __shared__ float mass_all[kReadWaves][kMaxCand];
  __shared__ int cand_all[kReadWaves][kMaxCand];
  __shared__ int sel_all[kReadWaves][kMaxCand];
  __shared__ float row_all[kReadWaves][D];
  float* mass_s = mass_all[w];                 // this wave's query scratch
  int* cand_id = cand_all[w];
  int* sel_id = sel_all[w];
  float* row_s = row_all[w];

  // Page z the tile sees, page weights and coarse weights (lanes = pages;
  // the waves take the channels in turn).
  const float* pzt = p.pz + bh * p.P8 * kGroup * D;
  for (int d = w; d < D; d += kReadWaves) {
    const float zp = lane < completed ? pzt[((size_t)lane * kGroup + kGroup - 1) * D + d]
                   : (lane == completed && pending)
                       ? pzt[((size_t)completed * kGroup + pending - 1) * D + d]
                       : -__builtin_inff();
    const float top = wave_max(zp);
    const float e = lane < P ? exp_cr(zp - top) : 0.0f;
    const float total = wave_fold(e);
    if (lane < P) pw[lane][d] = e / total;
    if (coarse_on) {
      const float zc = lane < completed ? zp : -__builtin_inff();
      const float tc = wave_max(zc);
      const float ec = lane < completed ? exp_cr(zc - tc) : 0.0f;
      const float tot = wave_fold(ec);
      if (lane < completed) cw[lane][d] = ec / tot;
    }
  }
  __syncthreads();

  const float* swt = p.swt + bh * p.P8 * kRowsPerPage * D;
  auto sw_row = [&](int id) -> const float* {
    const int pg = id / kGroup, j = id % kGroup;
    const int n = pg < completed ? kGroup : pending;
    return swt + ((size_t)pg * kRowsPerPage + n * (n - 1) / 2 + j) * D;
  };
  const float* bank = p.bank + bh * p.S * D * D;
  const float* pcb = p.pc ? p.pc + bh * p.Pc * D * D : nullptr;
  float a[R][3], fb[R][3];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int d = lane + 64 * r;
      a[r][i] = load_param(p.fa, p.f_dtype, h * p.fa_s[0] + d * p.fa_s[1] + i * p.fa_s[2]);
      fb[r][i] = load_param(p.fb, p.f_dtype, h * p.fb_s[0] + d * p.fb_s[1] + i * p.fb_s[2]);
    }

  for (int t = t0 + w; t < tend; t += kReadWaves) {
    // h = softmax over channels of raw_q
    float x[R], hq[R];
#pragma unroll
    for (int r = 0; r < R; ++r) x[r] = ld(p.rq, b, t, h, lane + 64 * r);
    float top = x[0];
    if constexpr (R == 2) top = fmaxf(x[0], x[1]);
    top = wave_max(top);
    float e[R];
#pragma unroll
    for (int r = 0; r < R; ++r) e[r] = exp_cr(x[r] - top);
    const float total = channel_fold<R>(e);
#pragma unroll
    for (int r = 0; r < R; ++r) hq[r] = e[r] / total;

    // Chosen pages: stable top-`coarse` of the completed pages' masses.
    int E = 0;
    if (coarse) {
      for (int pg = 0; pg < completed; ++pg) {
        float hv[R];
#pragma unroll
        for (int r = 0; r < R; ++r) hv[r] = hq[r] * pw[pg][lane + 64 * r];
        const float m = channel_fold<R>(hv);
        if (lane == 0) mass_s[pg] = m;
      }
      wave_sync();
      const bool mine = lane < completed;
      const int rank = mine ? stable_rank(mass_s[lane], lane, completed, mass_s) : kMaxCand;
      const bool chosen = rank < coarse;
      const unsigned long long bal = __ballot(chosen);
      const int pos = __popcll(bal & ((1ull << lane) - 1ull));
      wave_sync();
      if (chosen)
        for (int s = 0; s < kGroup; ++s) cand_id[pos * kGroup + s] = lane * kGroup + s;
      E = coarse * kGroup;
    }
    if (lane < pending) cand_id[E + lane] = completed * kGroup + lane;
    E += pending;
    wave_sync();

    // Candidate masses sum_d (h pw[page]) sw[fine], then the stable top-M.
    for (int c = 0; c < E; ++c) {
      const int id = cand_id[c];
      const int pg = id / kGroup;
      const float* sw = sw_row(id);
      float ch[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int d = lane + 64 * r;
        ch[r] = (hq[r] * pw[pg][d]) * sw[d];
      }
      const float m = channel_fold<R>(ch);
      if (lane == 0) mass_s[c] = m;
    }
    wave_sync();
    for (int c = lane; c < E; c += 64) {
      const int rank = stable_rank(mass_s[c], c, E, mass_s);
      if (rank < M) sel_id[rank] = cand_id[c];
    }
    wave_sync();
    if (p.sel_out)
      for (int m = lane; m < p.sel_cap; m += 64)
        p.sel_out[(((size_t)b * p.T + t) * p.H + h) * p.sel_cap + m] = m < M ? sel_id[m] : -1;

    // Selected read: num = sum_m ch_m C_m, den = butterfly over slots of the
    // butterfly channel sums; fine = num / den.
    float num[R] = {};
    float slot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int m = 0; m < M; ++m) {
      const int id = sel_id[m];
      const int pg = id / kGroup;
      const float* sw = sw_row(id);
      float ch[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int d = lane + 64 * r;
        ch[r] = (hq[r] * pw[pg][d]) * sw[d];
        row_s[d] = ch[r];
      }
      const float ps = channel_fold<R>(ch);
      if ((m & 63) == lane) slot[m >> 6] = ps;
      wave_sync();
      const float* c = bank + (size_t)id * D * D;
      for (int dd = 0; dd < D; ++dd) {
        const float w = row_s[dd];
#pragma unroll
        for (int r = 0; r < R; ++r) num[r] = fmaf(w, c[dd * D + lane + 64 * r], num[r]);
      }
      wave_sync();
    }
    const float den = slot_fold<4>(slot, M);
    float fine[R];
#pragma unroll
    for (int r = 0; r < R; ++r) fine[r] = num[r] / den;

    // Coarse read over the completed pages (coarse value branch).
    float coarse_v[R] = {};
    if (coarse_on) {
      for (int pg = 0; pg < completed; ++pg) {
#pragma unroll
        for (int r = 0; r < R; ++r) row_s[lane + 64 * r] = hq[r] * cw[pg][lane + 64 * r];
        wave_sync();
        const float* c = pcb + (size_t)pg * D * D;
        for (int dd = 0; dd < D; ++dd) {
          const float w = row_s[dd];
#pragma unroll
          for (int r = 0; r < R; ++r)
            coarse_v[r] = fmaf(w, c[dd * D + lane + 64 * r], coarse_v[r]);
        }
        wave_sync();
      }
    }

    // _fuse_training at fp32 (operator.py:21-38); both history branches
    // present only with coarse values past first_coarse.
    const float bias = coarse_on ? kLogTwoF32 : 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int d = lane + 64 * r;
      const float loc = local[(((size_t)b * p.T + t) * p.H + h) * D + d];
      float s[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) s[i] = (a[r][i] * x[r]) + fb[r][i];
      s[0] = s[0] + bias;
      if (!coarse_on) s[1] = -__builtin_inff();
      const float top3 = fmaxf(s[0], fmaxf(s[1], s[2]));
      const float e0 = exp_cr(s[0] - top3);
      const float e1 = coarse_on ? exp_cr(s[1] - top3) : 0.0f;
      const float e2 = exp_cr(s[2] - top3);
      const float tot = (e0 + e2) + e1;   // butterfly order over [e0, e1, e2, 0]
      const float r0 = e0 / tot, r1 = e1 / tot, r2 = e2 / tot;
      const float lt = r0 * (2.0f * loc);
      const float ct = r1 * (p.gain * coarse_v[r]);
      const float ft = r2 * (p.gain * fine[r]);
      *out_at(t, d) = (lt + ct) + ft;
    }
  }
}

}  // namespace

size_t f32_workspace_floats(int B, int H, int D, int64_t T, int coarse_values) {
  const int64_t tiles = (T + kFine - 1) / kFine;
  const int64_t S = tiles > 3 ? tiles - 3 : 0;
  const int64_t P8 = (S + kGroup - 1) / kGroup;
  const int64_t Pc = coarse_values ? S / kGroup : 0;
  const int64_t bh = (int64_t)B * H;
  auto align = [](int64_t n) { return (n + 63) & ~(int64_t)63; };
  return (size_t)(align(bh * T * D) + align(bh * S * D) + align(bh * S * D * D) +
                  align(bh * P8 * kGroup * D) + align(bh * P8 * kRowsPerPage * D) +
                  align(bh * Pc * D * D));
}

int f32_layout(F32Params& p, float* ws, int64_t T, int coarse_values) {
  const int64_t tiles = (T + kFine - 1) / kFine;
  p.S = (int)(tiles > 3 ? tiles - 3 : 0);
  p.P8 = (p.S + kGroup - 1) / kGroup;
  p.Pc = coarse_values ? p.S / kGroup : 0;
  p.T = (int)T;
  p.coarse_values = coarse_values;
  const int64_t bh = (int64_t)p.B * p.H;
  const int D = p.D;
  auto align = [](int64_t n) { return (n + 63) & ~(int64_t)63; };
  float* cur = ws;
  p.local = cur; cur += align(bh * T * D);
  p.fine_z = cur; cur += align(bh * p.S * D);
  p.bank = cur; cur += align(bh * (int64_t)p.S * D * D);
  p.pz = cur; cur += align(bh * p.P8 * kGroup * D);
  p.swt = cur; cur += align(bh * p.P8 * kRowsPerPage * D);
  p.pc = coarse_values && p.Pc ? cur : nullptr;
  return 0;
}

int f32_limits(const tao_stream_cfg& cfg, int64_t T, int64_t* pages, int64_t* cand) {
  const int64_t tiles = (T + kFine - 1) / kFine;
  const int64_t vmax = tiles > 3 ? tiles - 3 : 0;
  int64_t coarse = 0, elig = 0, sel = 0;
  if (vmax) sched::routed_counts(cfg, vmax / kGroup, vmax % kGroup, &coarse, &elig, &sel);
  *pages = vmax / kGroup + (vmax % kGroup > 0);
  *cand = coarse * kGroup + kGroup - 1;
  return *pages <= kMaxPages && *cand <= kMaxCand && sel <= kMaxCand;
}

hipError_t launch_full_f32(const F32Params& p, hipStream_t s, bool own_local) {
  const dim3 heads((unsigned)p.H, (unsigned)p.B);
  auto grid = [&](int64_t x) { return dim3((unsigned)x, heads.x, heads.y); };
  if (p.D == 64) {
    if (own_local)
      hipLaunchKernelGGL(f32_local_kernel<64>, grid((p.T + 63) / 64), dim3(64 * kLocalWaves<64>),
                         0, s, p);
    if (p.S) {
      hipLaunchKernelGGL(f32_writer_kernel<64>, grid(p.S), dim3(256), 0, s, p);
      hipLaunchKernelGGL(f32_pages_kernel<64>, grid(p.P8), dim3(64), 0, s, p);
    }
    hipLaunchKernelGGL(f32_read_kernel<64>, grid((p.T + kChunk - 1) / kChunk), dim3(64 * kReadWaves),
                       0, s, p);
  } else if (p.D == 128) {
    if (own_local)
      hipLaunchKernelGGL(f32_local_kernel<128>, grid((p.T + 63) / 64), dim3(64 * kLocalWaves<128>),
                         0, s, p);
    if (p.S) {
      hipLaunchKernelGGL(f32_writer_kernel<128>, grid(p.S), dim3(512), 0, s, p);
      hipLaunchKernelGGL(f32_pages_kernel<128>, grid(p.P8), dim3(128), 0, s, p);
    }
    hipLaunchKernelGGL(f32_read_kernel<128>, grid((p.T + kChunk - 1) / kChunk),
                       dim3(64 * kReadWaves), 0, s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace tao

namespace {

int f32_fail(int code, const char* msg) {
  tao::set_error(msg);
  return code;
}

tao::F32View f32_view(const void* p, const int64_t* s) {
  tao::F32View v;
  v.p = (const float*)p;
  v.sb = s[0];
  v.st = s[1];
  v.sh = s[2];
  return v;
}

}  // namespace

extern "C" {

size_t tao_full_sequence_f32_workspace_bytes(int32_t batch, int32_t heads, int32_t head_dim,
                                             int64_t tokens, int32_t coarse_values) {
  if (batch <= 0 || heads <= 0 || tokens < 0 || (head_dim != 64 && head_dim != 128)) return 0;
  return tao::f32_workspace_floats(batch, heads, head_dim, tokens, coarse_values ? 1 : 0) *
         sizeof(float);
}

}  // extern "C"

namespace {

// tao_full_sequence_f32 and tao_full_sequence_f32_local: local null computes
// the local attention, else the read takes it from `local`.
int full_f32(const tao_stream_cfg* cfg, const tao_tokens* tok, const tao_fusion* fu,
             int32_t batch, int32_t heads, int32_t head_dim, int32_t coarse_values,
             const void* local, void* out, const int64_t* out_s, int32_t* sel_out,
             int32_t sel_cap, void* workspace, size_t workspace_bytes, void* stream) {
  if (!cfg || !tok || !fu || !out || !out_s || !workspace)
    return f32_fail(TAO_E_ARGUMENT, "null fp32 full-sequence argument");
  if (!tok->q || !tok->k || !tok->v || !tok->raw_q || !tok->raw_k)
    return f32_fail(TAO_E_ARGUMENT, "null token operand");
  if (!fu->fusion_a || !fu->fusion_b ||
      (fu->dtype != TAO_BF16 && fu->dtype != TAO_FP32 && fu->dtype != TAO_FP16))
    return f32_fail(TAO_E_ARGUMENT, "invalid fusion parameters");
  if (cfg->fine_tokens != 256 || cfg->local_keep != 512 || cfg->coarse_group != 8)
    return f32_fail(TAO_E_ARGUMENT, "the fp32 read implements fine_tokens=256, local_keep=512, "
                                    "coarse_group=8");
  if (head_dim != 64 && head_dim != 128)
    return f32_fail(TAO_E_SHAPE, "head_dim must be 64 or 128");
  if (batch <= 0 || heads <= 0 || tok->tokens < 0)
    return f32_fail(TAO_E_SHAPE, "batch, heads and tokens must be positive");
  const int64_t T = tok->tokens;
  if (T == 0) return TAO_OK;
  if (T > (int64_t)1 << 30) return f32_fail(TAO_E_SHAPE, "sequence too long");
  int64_t pages = 0, cand = 0;
  if (!tao::f32_limits(*cfg, T, &pages, &cand))
    return f32_fail(TAO_E_CAPACITY, "the fp32 read holds at most 64 pages and 256 route "
                                    "candidates per query (sequence too long)");
  const size_t need = tao::f32_workspace_floats(batch, heads, head_dim, T, coarse_values ? 1 : 0) *
                      sizeof(float);
  if (sel_out && sel_cap <= 0) return f32_fail(TAO_E_ARGUMENT, "sel_out needs sel_cap > 0");
  if (workspace_bytes < need)
    return f32_fail(TAO_E_WORKSPACE, "workspace smaller than "
                                     "tao_full_sequence_f32_workspace_bytes()");
  tao::F32Params p{};
  p.q = f32_view(tok->q, tok->q_s);
  p.k = f32_view(tok->k, tok->k_s);
  p.v = f32_view(tok->v, tok->v_s);
  p.rq = f32_view(tok->raw_q, tok->rq_s);
  p.rk = f32_view(tok->raw_k, tok->rk_s);
  p.fa = fu->fusion_a;
  p.fb = fu->fusion_b;
  p.f_dtype = fu->dtype;
  for (int i = 0; i < 3; ++i) { p.fa_s[i] = fu->a_s[i]; p.fb_s[i] = fu->b_s[i]; }
  p.gain = fu->gain;
  p.out = (float*)out;
  p.out_sb = out_s[0];
  p.out_st = out_s[1];
  p.out_sh = out_s[2];
  p.sel_out = sel_out;
  p.sel_cap = sel_out ? sel_cap : 0;
  p.cfg = *cfg;
  p.B = batch;
  p.H = heads;
  p.D = head_dim;
  tao::f32_layout(p, (float*)workspace, T, coarse_values ? 1 : 0);
  if (local) p.local = const_cast<float*>((const float*)local);   // read only
  const hipError_t e = tao::launch_full_f32(p, (hipStream_t)stream, local == nullptr);
  if (e != hipSuccess) return f32_fail((int)e, hipGetErrorString(e));
  return TAO_OK;
}

}  // namespace

extern "C" {

int tao_full_sequence_f32(const tao_stream_cfg* cfg, const tao_tokens* tok, const tao_fusion* fu,
                          int32_t batch, int32_t heads, int32_t head_dim, int32_t coarse_values,
                          void* out, const int64_t* out_s, int32_t* sel_out, int32_t sel_cap,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return full_f32(cfg, tok, fu, batch, heads, head_dim, coarse_values, nullptr, out, out_s,
                  sel_out, sel_cap, workspace, workspace_bytes, stream);
}

int tao_full_sequence_f32_local(const tao_stream_cfg* cfg, const tao_tokens* tok,
                                const tao_fusion* fu, int32_t batch, int32_t heads,
                                int32_t head_dim, int32_t coarse_values, const void* local,
                                void* out, const int64_t* out_s, int32_t* sel_out,
                                int32_t sel_cap, void* workspace, size_t workspace_bytes,
                                void* stream) {
  if (!local) return f32_fail(TAO_E_ARGUMENT, "null local attention output");
  return full_f32(cfg, tok, fu, batch, heads, head_dim, coarse_values, local, out, out_s,
                  sel_out, sel_cap, workspace, workspace_bytes, stream);
}

}  // extern "C"
