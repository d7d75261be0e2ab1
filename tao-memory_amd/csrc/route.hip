// Routing refresh for gfx950: one workgroup per (batch, head).
//
// Restates tao_stream.py:310-357 with _topk_oldest (:50-53):
//   h    = r(softmax_D(raw_q))                 (anchor query row)
//   hv_p = r(h * pw[p])                        (page weights of the epoch)
//   page mass = r(sum_D hv_p) over completed pages; stable top-`coarse`
//   pages (descending, lowest index wins ties), re-sorted ascending;
//   candidates = 8 fines of each chosen page + every pending fine;
//   mass_j = r(sum_D r(hv_page(j) * sw_j)); stable top-M candidates kept in
//   score order.
// Every fp32 sum uses the butterfly order of the oracle, so selected ids are
// bit-identical to the oracle's. Selection: 64-bit keys (monotone bf16 score
// << 32 | ~index) ranked by counting (<= 512 keys) or an LDS bitonic network.
// Eight waves issue the loads of eight rows each before reducing them, so a
// refresh costs a few memory latencies rather than one per row.
#include "tao_launch.h"
#include "tao_common.h"

namespace tao {
namespace {

constexpr int kMaxSort = 2048;   // pages or candidates per head

template <int D>
struct RouteSmem {
  float h[D];
  unsigned long long keys[kMaxSort];
  int cand_id[kMaxSort];
  int cand_page[kMaxSort];
  int chosen[kMaxSort / 8];
};

TAO_DEV unsigned long long score_key(float score_bf, int index) {
  bf16_t bits = f2bf(score_bf);
  if (bits == 0x8000) bits = 0;      // -0 ties with +0, as in torch's sort
  const uint32_t hi = bf16_order_key(bits);
  return ((unsigned long long)hi << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)index);
}

TAO_DEV int key_index(unsigned long long key) {
  return (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
}

constexpr int kRouteThreads = 512;   // 8 waves
constexpr int kWaves = kRouteThreads / 64;
constexpr int kBatch = 8;            // rows whose loads one wave issues together
constexpr int kRankMax = 512;        // rank-count selection up to this many keys

// Masses of up to kBatch rows per wave: every lane loads its two (or one)
// channels of all rows first, then each row is reduced in butterfly order:
// r(sum_D r(h * pw[page]) [* sw[id]]).
// Segment-weight rows: fines below `split` read the state's final weights,
// later (pending) fines read the epoch's pool rows.
struct SwRows {
  const bf16_t* lo; const bf16_t* hi; int split;
  TAO_DEV const bf16_t* row(int id, int D) const {
    return id < split ? lo + (size_t)id * D : hi + (size_t)(id - split) * D;
  }
};

template <int D>
TAO_DEV void wave_masses(const float* h, const bf16_t* pw, const SwRows* sw,
                         const int* pages, const int* ids, int count, int lane,
                         float* out) {
  constexpr int PER = D / 64;
  bf16_t pv[kBatch][PER], sv[kBatch][PER];
#pragma unroll
  for (int r = 0; r < kBatch; ++r) {
    if (r < count) {
      const bf16_t* srow = sw ? sw->row(ids[r], D) : nullptr;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        pv[r][k] = pw[(size_t)pages[r] * D + lane + 64 * k];
        sv[r][k] = sw ? srow[lane + 64 * k] : (bf16_t)0;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kBatch; ++r) {
    if (r < count) {
      float v[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const float hv = rbf(h[lane + 64 * k] * bf2f(pv[r][k]));
        v[k] = sw ? rbf(hv * bf2f(sv[r][k])) : hv;
      }
      float s = v[0];
#pragma unroll
      for (int k = 1; k < PER; ++k) s += v[k];
      out[r] = rbf(wave_sum_fold(s));
    }
  }
}

// h = r(softmax_D(raw_q row)) of one query by one wave: fp32 exp correctly
// rounded, butterfly sum (tao_stream.py:253-254).
template <int D>
TAO_DEV void query_weights(const bf16_t* rq, int lane, float* h) {
  constexpr int PER = D / 64;
  float x[PER], e[PER];
  float mx = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < PER; ++k) { x[k] = bf2f(rq[lane + 64 * k]); mx = fmaxf(mx, x[k]); }
  mx = wave_max(mx);
#pragma unroll
  for (int k = 0; k < PER; ++k) e[k] = exp_cr(x[k] - mx);
  float s = e[0];
#pragma unroll
  for (int k = 1; k < PER; ++k) s += e[k];
  s = wave_sum_fold(s);
#pragma unroll
  for (int k = 0; k < PER; ++k) h[lane + 64 * k] = rbf(e[k] / s);
}

// Stable descending selection of the top `count` keys (unique 64-bit keys:
// score << 32 | ~index). Writes the selected keys, best first, to dst.
__device__ void select_top(unsigned long long* keys, int n, int count,
                           unsigned long long* dst) {
  if (n <= kRankMax) {
    for (int i = threadIdx.x; i < n; i += kRouteThreads) {
      const unsigned long long mine = keys[i];
      int rank = 0;
      for (int j = 0; j < n; ++j) rank += keys[j] > mine;
      if (rank < count) dst[rank] = mine;
    }
    __syncthreads();
    return;
  }
  int np = 1;
  while (np < n) np <<= 1;
  for (int i = n + threadIdx.x; i < np; i += kRouteThreads) keys[i] = 0ull;
  __syncthreads();
  for (int k = 2; k <= np; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < np; i += kRouteThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const unsigned long long a = keys[i], b = keys[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (a < b) : (a > b)) { keys[i] = b; keys[ixj] = a; }
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < count; i += kRouteThreads) dst[i] = keys[i];
  __syncthreads();
}

template <int D>
__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteParams p) {
  __shared__ RouteSmem<D> sm;
  __shared__ unsigned long long top[kMaxSort];
  constexpr int PER = D / 64;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Turn description (single-turn mode: the state's current epoch).
  long long anchor = 0;
  int K = p.completed, pending = p.pending, coarse = p.coarse, selected = p.selected;
  int write_state = 1;
  int32_t* sel_out = p.sel + (size_t)bh * p.sel_cap;
  const bf16_t* pw = p.pw + (size_t)bh * p.page_cap * D;
  SwRows swr{p.sw + (size_t)bh * p.fine_cap * D, nullptr, 0x7FFFFFFF};
  if (p.turns) {
    const int64_t* t = p.turns + 8 * (blockIdx.x / BH);
    anchor = t[0];
    const int erel = (int)t[1];
    K = (int)t[2]; pending = (int)t[3]; coarse = (int)t[4]; selected = (int)t[5];
    sel_out = p.sel_pool + ((size_t)t[6] * BH + bh) * p.sel_cap;
    write_state = (int)t[7];
    pw = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
    swr.hi = p.psw_pool + ((size_t)erel * BH + bh) * 8 * D;
    swr.split = K * p.group;
  }

  if (wave == 0) query_weights<D>(p.rq + b * p.rq_sb + anchor * p.rq_st + h * p.rq_sh, lane, sm.h);
  __syncthreads();

  // ---- coarse pages: stable top-`coarse` by page mass, then ascending.
  if (coarse > 0) {
    for (int base = wave * kBatch; base < K; base += kWaves * kBatch) {
      int pages[kBatch];
      float mass[kBatch];
      const int count = min(kBatch, K - base);
#pragma unroll
      for (int r = 0; r < kBatch; ++r) pages[r] = base + min(r, count - 1);
      wave_masses<D>(sm.h, pw, nullptr, pages, pages, count, lane, mass);
      if (lane < count) {
        float mine = mass[0];
#pragma unroll
        for (int r = 1; r < kBatch; ++r) if (lane == r) mine = mass[r];
        sm.keys[base + lane] = score_key(mine, base + lane);
      }
    }
    __syncthreads();
    select_top(sm.keys, K, coarse, top);
    if (tid < coarse) {
      const int mine = key_index(top[tid]);
      int rank = 0;
      for (int j = 0; j < coarse; ++j) rank += key_index(top[j]) < mine;
      sm.chosen[rank] = mine;
    }
    __syncthreads();
  }

  // ---- candidates: 8 fines of each chosen page, then the pending fines.
  const int group = p.group;
  const int E = group * coarse + pending;
  for (int j = tid; j < E; j += kRouteThreads) {
    int page, id;
    if (j < group * coarse) {
      page = sm.chosen[j / group];
      id = page * group + j % group;
    } else {
      page = K;
      id = K * group + (j - group * coarse);
    }
    sm.cand_page[j] = page;
    sm.cand_id[j] = id;
  }
  __syncthreads();
  for (int base = wave * kBatch; base < E; base += kWaves * kBatch) {
    int pages[kBatch], ids[kBatch];
    float mass[kBatch];
    const int count = min(kBatch, E - base);
#pragma unroll
    for (int r = 0; r < kBatch; ++r) {
      const int j = base + min(r, count - 1);
      pages[r] = sm.cand_page[j];
      ids[r] = sm.cand_id[j];
    }
    wave_masses<D>(sm.h, pw, &swr, pages, ids, count, lane, mass);
    if (lane < count) {
      float mine = mass[0];
#pragma unroll
      for (int r = 1; r < kBatch; ++r) if (lane == r) mine = mass[r];
      sm.keys[base + lane] = score_key(mine, base + lane);
    }
  }
  __syncthreads();
  select_top(sm.keys, E, selected, top);
  for (int m = tid; m < selected; m += kRouteThreads) {
    const int id = sm.cand_id[key_index(top[m])];
    sel_out[m] = id;
    if (write_state && p.turns) p.sel[(size_t)bh * p.sel_cap + m] = id;
  }
  if (write_state)
    for (int i = tid; i < coarse; i += kRouteThreads)
      p.chosen[(size_t)bh * p.chosen_cap + i] = sm.chosen[i];
  if (write_state && bh == 0 && tid == 0) p.header[1] = selected;
}

// ---------------------------------------------------------------------------
// Per-query routes of the full-sequence read (route_interval = 1 in
// _read_training_group, tao_stream.py:596-665, with candidate_scores,
// routing_scores.py:7-47): every history query of a read tile routes itself
// against its tile's epoch with route_kernel's arithmetic and reduction
// order (same candidates, masses and stable top-k), and its selection is
// written as a bitmask over fine ids; the read needs the set, not the order.
// One 256-thread workgroup per (read tile, batch, head); wave w routes
// queries w, w + 4, ... of the tile. Every wave runs the same number of
// rounds, so the barriers that publish its LDS keys are workgroup-uniform.
constexpr int kQThreads = 256;
constexpr int kQWaves = kQThreads / 64;
constexpr int kQMaxWords = 512;          // bitmask words per query (16384 fines)

template <int D>
struct QueryRouteSmem {
  float h[kQWaves][D];
  unsigned long long keys[kQWaves][kQueryRouteMaxKeys];
  int chosen[kQWaves][kQueryRouteMaxKeys / 8];
  uint32_t bits[kQWaves][kQMaxWords];
};

// Number of keys larger than `mine` among keys[0, n) (keys are unique).
TAO_DEV int key_rank(const unsigned long long* keys, int n, unsigned long long mine) {
  int r = 0;
  for (int j = 0; j < n; ++j) r += keys[j] > mine;
  return r;
}

template <int D>
__global__ __launch_bounds__(kQThreads) void route_queries_kernel(QueryRouteParams p) {
  __shared__ QueryRouteSmem<D> sm;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int b = bh / p.H, h = bh % p.H;
  const int64_t* desc = p.tiles + 8 * (blockIdx.x / BH);
  if (!desc[6]) return;                          // no history: workgroup-uniform
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int q_first = (int)desc[0], nq = (int)desc[1];
  const int coarse = (int)desc[2], M = (int)desc[3], erel = (int)desc[4];
  const int G = p.group;
  const int epoch = p.first_epoch + erel;
  const int K = epoch / G, pending = epoch % G;
  const int E = G * coarse + pending;
  const int words = (epoch + 31) >> 5;
  const bf16_t* pw = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
  const SwRows swr{p.sw + (size_t)bh * p.fine_cap * D,
                   p.psw_pool + ((size_t)erel * BH + bh) * 8 * D, K * G};
  float* hw = sm.h[w];
  unsigned long long* keys = sm.keys[w];
  int* chosen = sm.chosen[w];
  uint32_t* bits = sm.bits[w];
  auto cand = [&](int j, int& page, int& id) __attribute__((always_inline)) {
    if (j < G * coarse) {
      page = chosen[j / G];
      id = page * G + j % G;
    } else {
      page = K;
      id = K * G + (j - G * coarse);
    }
  };
  const int rounds = (nq + kQWaves - 1) / kQWaves;
  for (int r = 0; r < rounds; ++r) {
    const int qi = r * kQWaves + w;
    const bool on = qi < nq;
    const int t = q_first + (on ? qi : 0);
    if (on) query_weights<D>(p.rq + b * p.rq_sb + (int64_t)t * p.rq_st + h * p.rq_sh, lane, hw);
    for (int i = lane; i < words; i += 64) bits[i] = 0u;
    __syncthreads();
    // ---- page masses of the completed pages
    if (on && coarse > 0)
      for (int base = 0; base < K; base += kBatch) {
        int pages[kBatch];
        float mass[kBatch];
        const int count = min(kBatch, K - base);
#pragma unroll
        for (int i = 0; i < kBatch; ++i) pages[i] = base + min(i, count - 1);
        wave_masses<D>(hw, pw, nullptr, pages, pages, count, lane, mass);
        if (lane < count) {
          float mine = mass[0];
#pragma unroll
          for (int i = 1; i < kBatch; ++i) if (lane == i) mine = mass[i];
          keys[base + lane] = score_key(mine, base + lane);
        }
      }
    __syncthreads();
    // ---- stable top-`coarse` pages, listed ascending
    if (on && coarse > 0) {
      int placed = 0;
      for (int c0 = 0; c0 < K; c0 += 64) {
        const int i = c0 + lane;
        const bool pick = i < K && key_rank(keys, K, keys[i]) < coarse;
        const unsigned long long ball = __ballot(pick);
        if (pick) chosen[placed + __popcll(ball & ((1ull << lane) - 1ull))] = i;
        placed += __popcll(ball);
      }
    }
    __syncthreads();
    // ---- candidate masses: 8 fines of each chosen page, then the pending fines
    if (on)
      for (int base = 0; base < E; base += kBatch) {
        int pages[kBatch], ids[kBatch];
        float mass[kBatch];
        const int count = min(kBatch, E - base);
#pragma unroll
        for (int i = 0; i < kBatch; ++i) cand(base + min(i, count - 1), pages[i], ids[i]);
        wave_masses<D>(hw, pw, &swr, pages, ids, count, lane, mass);
        if (lane < count) {
          float mine = mass[0];
#pragma unroll
          for (int i = 1; i < kBatch; ++i) if (lane == i) mine = mass[i];
          keys[base + lane] = score_key(mine, base + lane);
        }
      }
    __syncthreads();
    // ---- stable top-M candidates -> bitmask
    if (on)
      for (int j = lane; j < E; j += 64)
        if (key_rank(keys, E, keys[j]) < M) {
          int page, id;
          cand(j, page, id);
          atomicOr(&bits[id >> 5], 1u << (id & 31));
        }
    __syncthreads();
    if (on) {
      uint32_t* dst = p.qsel + ((size_t)(b * p.T + t) * p.H + h) * p.qsel_words;
      for (int i = lane; i < words; i += 64) dst[i] = bits[i];
    }
    __syncthreads();                             // h, keys and bits are reused
  }
}

}  // namespace

hipError_t launch_route_queries(const QueryRouteParams& p, int head_dim, hipStream_t s) {
  if (p.n_tiles <= 0) return hipSuccess;
  if (p.qsel_words < 1 || p.qsel_words > kQMaxWords || p.group != 8)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)(p.n_tiles * p.B * p.H));
  if (head_dim == 128)
    hipLaunchKernelGGL(route_queries_kernel<128>, grid, dim3(kQThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(route_queries_kernel<64>, grid, dim3(kQThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_route(const RouteParams& p, int head_dim, hipStream_t s) {
  if (p.completed > kMaxSort || p.group * p.coarse + p.pending > kMaxSort)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)(p.B * p.H * (p.turns ? p.n_turns : 1)));
  if (head_dim == 128)
    hipLaunchKernelGGL(route_kernel<128>, grid, dim3(kRouteThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(route_kernel<64>, grid, dim3(kRouteThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace tao
