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
// Every fp32 sum uses the butterfly order of the oracle (wave_fold_sum: DPP
// on the bit-reversed channel layout), so selected ids are bit-identical to
// the oracle's. Selection: 64-bit keys (monotone bf16 score
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
constexpr int kRefreshThreads = 1024;   // the refresh: 16 waves per (batch, head)
constexpr int kRefreshWaves = kRefreshThreads / 64;
constexpr int kRefreshRowsPerWave = 5;   // staged rows one refresh wave reduces together
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
  const int e0 = fold_lane(lane);      // channels e0 + 64 k (bit-reversed layout)
  bf16_t pv[kBatch][PER], sv[kBatch][PER];
#pragma unroll
  for (int r = 0; r < kBatch; ++r) {
    if (r < count) {
      const bf16_t* srow = sw ? sw->row(ids[r], D) : nullptr;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        pv[r][k] = pw[(size_t)pages[r] * D + e0 + 64 * k];
        sv[r][k] = sw ? srow[e0 + 64 * k] : (bf16_t)0;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kBatch; ++r) {
    if (r < count) {
      float v[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const float hv = rbf(h[e0 + 64 * k] * bf2f(pv[r][k]));
        v[k] = sw ? rbf(hv * bf2f(sv[r][k])) : hv;
      }
      float s = v[0];
#pragma unroll
      for (int k = 1; k < PER; ++k) s += v[k];
      out[r] = rbf(wave_fold_sum(s));
    }
  }
}

// h = r(softmax_D(raw_q row)) of one query by one wave: fp32 exp correctly
// rounded, butterfly sum (tao_stream.py:253-254).
template <int D>
TAO_DEV void query_weights(const bf16_t* rq, int lane, float* h) {
  constexpr int PER = D / 64;
  const int e0 = fold_lane(lane);      // channels e0 + 64 k (bit-reversed layout)
  float x[PER], e[PER];
  float mx = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < PER; ++k) { x[k] = bf2f(rq[e0 + 64 * k]); mx = fmaxf(mx, x[k]); }
  mx = wave_fold_max(mx);
#pragma unroll
  for (int k = 0; k < PER; ++k) e[k] = exp_cr(x[k] - mx);
  float s = e[0];
#pragma unroll
  for (int k = 1; k < PER; ++k) s += e[k];
  s = wave_fold_sum(s);
#pragma unroll
  for (int k = 0; k < PER; ++k) h[e0 + 64 * k] = rbf(e[k] / s);
}

// Number of keys larger than `mine` among keys[0, n) (keys are unique).
TAO_DEV int key_rank(const unsigned long long* keys, int n, unsigned long long mine) {
  int r = 0;
  int j = 0;
  for (; j + 8 <= n; j += 8) {
    unsigned long long k8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) k8[i] = keys[j + i];
#pragma unroll
    for (int i = 0; i < 8; ++i) r += k8[i] > mine;
  }
  for (; j < n; ++j) r += keys[j] > mine;
  return r;
}

// Stable descending selection of the top `count` keys (unique 64-bit keys:
// score << 32 | ~index) by a workgroup of NT threads. Writes the selected
// keys, best first, to dst.
template <int NT>
TAO_DEV void select_top_n(unsigned long long* keys, int n, int count, unsigned long long* dst) {
  if (n <= 2 * NT / 8) {
    // T lanes per key (8 for n <= NT / 8, else 4): lane part p counts the
    // larger keys among keys p, p + T, ... (four reads in flight at a time;
    // 0 is below every key); DPP adds the T parts.
    const int T = n <= NT / 8 ? 8 : 4;
    const int i = threadIdx.x / T, part = threadIdx.x % T;
    const unsigned long long mine = keys[min(i, n - 1)];
    int cnt = 0;
    for (int j0 = part; j0 < n; j0 += 4 * T) {
      unsigned long long k4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) k4[u] = j0 + u * T < n ? keys[j0 + u * T] : 0ull;
#pragma unroll
      for (int u = 0; u < 4; ++u) cnt += k4[u] > mine;
    }
    cnt += __builtin_amdgcn_update_dpp(0, cnt, 0xB1, 0xF, 0xF, false);
    cnt += __builtin_amdgcn_update_dpp(0, cnt, 0x4E, 0xF, 0xF, false);
    if (T == 8) cnt += __builtin_amdgcn_update_dpp(0, cnt, 0x141, 0xF, 0xF, false);
    if (i < n && part == 0 && cnt < count) dst[cnt] = mine;
    __syncthreads();
    return;
  }
  if (n <= kRankMax) {
    for (int i = threadIdx.x; i < n; i += NT) {
      const unsigned long long mine = keys[i];
      const int rank = key_rank(keys, n, mine);
      if (rank < count) dst[rank] = mine;
    }
    __syncthreads();
    return;
  }
  int np = 1;
  while (np < n) np <<= 1;
  for (int i = n + threadIdx.x; i < np; i += NT) keys[i] = 0ull;
  __syncthreads();
  for (int k = 2; k <= np; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < np; i += NT) {
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
  for (int i = threadIdx.x; i < count; i += NT) dst[i] = keys[i];
  __syncthreads();
}

TAO_DEV void select_top(unsigned long long* keys, int n, int count, unsigned long long* dst) {
  select_top_n<kRouteThreads>(keys, n, count, dst);
}

template <int D>
__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteParams p) {
  __shared__ RouteSmem<D> sm;
  __shared__ unsigned long long top[kMaxSort];
  if (gate_closed(p.gate)) return;   // uniform: every thread reads one header word
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
// Single-turn refresh of a stream (the decode driver's route turns) with its
// rows staged in LDS: the same arithmetic, candidate order, butterfly sums
// and stable selections as route_kernel, but every row is fetched with
// coalesced 16-byte loads into LDS, so a refresh costs two memory round
// trips: (1) the page weights of the completed and pending pages, the
// pending fines' segment weights and the anchor query; (2) the segment
// weights of the chosen pages' fines. Serves states with at most
// kRefreshPages pages and kRefreshRows candidates; route_kernel serves the
// rest.
constexpr int kRefreshPages = 128;
constexpr int kRefreshRows = 128;

template <int D>
struct RefreshSmem {
  bf16_t pw[kRefreshPages][D];         // page weights, completed then pending page
  bf16_t sw[kRefreshRows][D];          // segment weights of the candidates, in order
  float h[D];
  unsigned long long keys[kRefreshRows];
  unsigned long long top[kRefreshRows];
  int chosen[kRefreshRows / 8 + 1];
};

// Masses of kBatch staged rows on one wave (bit-reversed channel layout,
// the butterfly sum of wave_masses): r(sum_D r(h * pw_row) [* sw_row]).
// The rows' reductions are independent and unrolled, so their latencies
// overlap. Rows past `count` (wave-uniform) give 0 and are not used; this
// wave's lane r < count receives row r's mass.
template <int D, int NB>
TAO_DEV float staged_masses(const float* h, const bf16_t* const* pw_rows,
                            const bf16_t* const* sw_rows, int count, int lane) {
  constexpr int PER = D / 64;
  const int e0 = fold_lane(lane);
  float hq[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) hq[k] = h[e0 + 64 * k];
  // Rows past `count` repeat the last row (callers clamp), so every read is
  // unconditional and the reads of all rows are in flight together.
  bf16_t pv[NB][PER], sv[NB][PER];
#pragma unroll
  for (int r = 0; r < NB; ++r)
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      pv[r][k] = pw_rows[r][e0 + 64 * k];
      sv[r][k] = sw_rows ? sw_rows[r][e0 + 64 * k] : (bf16_t)0;
    }
  float part[NB];
#pragma unroll
  for (int r = 0; r < NB; ++r) {
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const float hv = rbf(hq[k] * bf2f(pv[r][k]));
      v[k] = sw_rows ? rbf(hv * bf2f(sv[r][k])) : hv;
    }
    float s = v[0];
#pragma unroll
    for (int k = 1; k < PER; ++k) s += v[k];
    part[r] = s;
  }
  wave_fold_sum_n<NB>(part);
  float mine = 0.0f;
#pragma unroll
  for (int r = 0; r < NB; ++r)
    if (lane == r) mine = rbf(part[r]);
  (void)count;
  return mine;
}

// The refresh's selection for (batch, head) bh by a workgroup of NT
// threads: the route of RouteParams' single turn, left in LDS (sm.top: the
// selected candidates' keys, best first; sm.chosen: the chosen pages,
// ascending; sm.pw / sm.sw: the page weights and the candidates' segment
// weights). Each mass is a butterfly sum inside one wave, so the result does
// not depend on NT. With `write_out` the selection is also stored in the
// state (sel, chosen; header[1] by head 0).
template <int D, int NT>
TAO_DEV void refresh_select(const RouteParams& p, int bh, RefreshSmem<D>& sm, bool write_out) {
  constexpr int C16 = D / 8;            // 16-byte chunks per row
  constexpr int NW = NT / 64;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = p.completed, pending = p.pending, coarse = p.coarse, selected = p.selected;
  constexpr int group = 8;          // coarse_group (checked at launch)
  const int P = K + (pending > 0 ? 1 : 0);
  const int E = group * coarse + pending;
  const bf16_t* pw = p.pw + (size_t)bh * p.page_cap * D;
  const bf16_t* sw = p.sw + (size_t)bh * p.fine_cap * D;
  // ---- round trip 1: page weights, pending segment weights, anchor query
  // (every load issued before any store to LDS)
  constexpr int PW_PT = (kRefreshPages * C16 + NT - 1) / NT;
  constexpr int SW_PT = (kRefreshRows * C16 + NT - 1) / NT;
  constexpr int PD_PT = (8 * C16 + NT - 1) / NT;   // pending fines: fewer than 8 rows
  // Loads are unconditional (indices clamped to a valid row) so the
  // scheduler can issue them all before the guarded LDS stores.
  uint4 pwv[PW_PT], pdv[PD_PT];
#pragma unroll
  for (int k = 0; k < PW_PT; ++k) {
    const int ic = min(tid + k * NT, P * C16 - 1);
    pwv[k] = *(const uint4*)(pw + (size_t)(ic / C16) * D + (ic % C16) * 8);
  }
  if (pending > 0) {
#pragma unroll
    for (int k = 0; k < PD_PT; ++k) {
      const int ic = min(tid + k * NT, pending * C16 - 1);
      pdv[k] = *(const uint4*)(sw + (size_t)(K * group + ic / C16) * D + (ic % C16) * 8);
    }
  }
#pragma unroll
  for (int k = 0; k < PW_PT; ++k) {
    const int i = tid + k * NT;
    if (i < P * C16) *(uint4*)&sm.pw[i / C16][(i % C16) * 8] = pwv[k];
  }
  if (pending > 0) {
#pragma unroll
    for (int k = 0; k < PD_PT; ++k) {
      const int i = tid + k * NT;
      if (i < pending * C16) *(uint4*)&sm.sw[group * coarse + i / C16][(i % C16) * 8] = pdv[k];
    }
  }
  if (wave == 0) query_weights<D>(p.rq + b * p.rq_sb + h * p.rq_sh, lane, sm.h);
  __syncthreads();
  // ---- coarse pages: stable top-`coarse` by page mass, then ascending
  if (coarse > 0) {
    for (int base = wave * kRefreshRowsPerWave; base < K; base += NW * kRefreshRowsPerWave) {
      const int count = min(kRefreshRowsPerWave, K - base);
      const bf16_t* rows[kRefreshRowsPerWave];
#pragma unroll
      for (int r = 0; r < kRefreshRowsPerWave; ++r) rows[r] = sm.pw[base + min(r, count - 1)];
      const float mass = staged_masses<D, kRefreshRowsPerWave>(sm.h, rows, nullptr, count, lane);
      if (lane < count) sm.keys[base + lane] = score_key(mass, base + lane);
    }
    __syncthreads();
    select_top_n<NT>(sm.keys, K, coarse, sm.top);
    if (tid < coarse) {
      const int mine = key_index(sm.top[tid]);
      int rank = 0;
      for (int j = 0; j < coarse; ++j) rank += key_index(sm.top[j]) < mine;
      sm.chosen[rank] = mine;
    }
    __syncthreads();
    // ---- round trip 2: segment weights of the chosen pages' fines
    uint4 swv[SW_PT];
#pragma unroll
    for (int k = 0; k < SW_PT; ++k) {
      const int ic = min(tid + k * NT, group * coarse * C16 - 1);
      const int row = ic / C16;
      const int id = sm.chosen[row / group] * group + row % group;
      swv[k] = *(const uint4*)(sw + (size_t)id * D + (ic % C16) * 8);
    }
#pragma unroll
    for (int k = 0; k < SW_PT; ++k) {
      const int i = tid + k * NT;
      if (i < group * coarse * C16) *(uint4*)&sm.sw[i / C16][(i % C16) * 8] = swv[k];
    }
    __syncthreads();
  }
  // ---- candidate masses: 8 fines of each chosen page, then the pending fines
  for (int base = wave * kRefreshRowsPerWave; base < E; base += NW * kRefreshRowsPerWave) {
    const int count = min(kRefreshRowsPerWave, E - base);
    const bf16_t* prow[kRefreshRowsPerWave];
    const bf16_t* srow[kRefreshRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRefreshRowsPerWave; ++r) {
      const int j = base + min(r, count - 1);
      prow[r] = sm.pw[j < group * coarse ? sm.chosen[j / group] : K];
      srow[r] = sm.sw[j];
    }
    const float mass = staged_masses<D, kRefreshRowsPerWave>(sm.h, prow, srow, count, lane);
    if (lane < count) sm.keys[base + lane] = score_key(mass, base + lane);
  }
  __syncthreads();
  select_top_n<NT>(sm.keys, E, selected, sm.top);
  if (!write_out) return;
  int32_t* sel_out = p.sel + (size_t)bh * p.sel_cap;
  for (int m = tid; m < selected; m += NT) {
    const int j = key_index(sm.top[m]);
    sel_out[m] = j < group * coarse ? sm.chosen[j / group] * group + j % group
                                    : K * group + (j - group * coarse);
  }
  for (int i = tid; i < coarse; i += NT)
    p.chosen[(size_t)bh * p.chosen_cap + i] = sm.chosen[i];
  if (bh == 0 && tid == 0) p.header[1] = selected;
}

template <int D>
__global__ __launch_bounds__(kRefreshThreads) void route_refresh_kernel(RouteParams p) {
  __shared__ RefreshSmem<D> sm;
  if (gate_closed(p.gate)) return;   // uniform: every thread reads one header word
  refresh_select<D, kRefreshThreads>(p, blockIdx.x, sm, true);
}

// Route refresh and fold in one launch: the fold's CHUNKS workgroups of a
// (batch, head) each compute the head's selection (refresh_select on 16
// waves; the same arithmetic gives every workgroup the same route, and
// chunk 0 stores it), then fold their ROWS rows of G^T over the selected
// fines with fold_kernel's arithmetic and order: in slot order m, w_m[d] =
// pw[page(m)][d] * sw[m][d] (from the rows the selection staged in LDS,
// kRefreshFoldStage slots at a time), G^T[e][d] += w_m[d] * C^T_m[e][d] as
// one fp32 FMA, g[d] += w_m[d]. Thread (row, column pair) loads 4 bytes of
// each selected C^T row, so a wave reads one 256-byte row per slot. One
// launch instead of two removes a launch gap and the fold's wait for the
// route kernel's last workgroup.
constexpr int kRefreshFoldStage = 36;

template <int D>
__global__ __launch_bounds__(kRefreshThreads) void refresh_fold_kernel(RouteParams p,
                                                                        FoldParams f) {
  constexpr int NT = kRefreshThreads;
  constexpr int CP = D / 2, ROWS = NT / CP, CHUNKS = D / ROWS, U = kRefreshFoldStage;
  constexpr int group = 8;
  __shared__ RefreshSmem<D> sm;
  __shared__ float wts[U][D];
  __shared__ int slot_id[U];
  if (gate_closed(p.gate)) return;   // uniform: every thread reads one header word
  int bh, e_chunk;
  xcd_unit(blockIdx.x, p.B * p.H, CHUNKS, bh, e_chunk);
  refresh_select<D, NT>(p, bh, sm, e_chunk == 0);
  const int tid = threadIdx.x, cp = tid % CP, r = tid / CP;
  const int e = e_chunk * ROWS + r;
  const int K = p.completed, coarse = p.coarse, M = p.selected;
  const bf16_t* bank = f.bank + (size_t)bh * f.fine_cap * D * D;
  float acc0 = 0.0f, acc1 = 0.0f, den0 = 0.0f, den1 = 0.0f;
  for (int s0 = 0; s0 < M; s0 += U) {
    const int staged = min(U, M - s0);
    __syncthreads();                  // the previous stage is consumed (or the selection done)
    if (tid < staged) {
      const int j = key_index(sm.top[s0 + tid]);
      slot_id[tid] = j < group * coarse ? sm.chosen[j / group] * group + j % group
                                        : K * group + (j - group * coarse);
    }
    __syncthreads();
    // The stage's C^T loads first, then its weights (slot u's page row and
    // candidate row, both staged) while the loads are in flight.
    uint32_t cv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int m = min(u, staged - 1);
      cv[u] = *(const uint32_t*)(bank + ((size_t)slot_id[m] * D + e) * D + cp * 2);
    }
    for (int i = tid; i < staged * D; i += NT) {
      const int u = i / D, d = i % D;
      const int j = key_index(sm.top[s0 + u]);
      const int prow = j < group * coarse ? sm.chosen[j / group] : K;
      wts[u][d] = bf2f(sm.pw[prow][d]) * bf2f(sm.sw[j][d]);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (u < staged) {
        const float2 w = *(const float2*)&wts[u][cp * 2];
        acc0 = fmaf(w.x, __uint_as_float(cv[u] << 16), acc0);
        acc1 = fmaf(w.y, __uint_as_float(cv[u] & 0xFFFF0000u), acc1);
        den0 += w.x;
        den1 += w.y;
      }
    }
  }
  *(float2*)(f.fold_g + ((size_t)bh * D + e) * D + cp * 2) = make_float2(acc0, acc1);
  if (e == 0) *(float2*)(f.fold_den + (size_t)bh * D + cp * 2) = make_float2(den0, den1);
}

// ---------------------------------------------------------------------------
// Per-query routes of the full-sequence read (route_interval = 1 in
// _read_training_group, tao_stream.py:596-665, with candidate_scores,
// routing_scores.py:7-47): every history query of a read tile routes itself
// against its tile's epoch with route_kernel's arithmetic and reduction
// order (same candidates, masses and stable top-k), and its selection is
// written as a bitmask over fine ids; the read needs the set, not the order.
// One 256-thread workgroup per (read tile, batch, head); wave w routes
// queries w, w + 4, ... on its own LDS arrays, so waves only synchronise
// with themselves. This is the general path (any number of visible fines up
// to the read's limit); route_tile_kernel below serves tiles whose rows fit
// in LDS.
constexpr int kQThreads = 256;
constexpr int kQWaves = kQThreads / 64;
constexpr int kQMaxWords = 512;          // bitmask words per query (16384 fines)

template <int D>
struct QueryRouteSmem {
  float h[kQWaves][D];
  unsigned long long keys[kQWaves][kQueryRouteMaxKeys];
  int chosen[kQWaves][kQueryRouteMaxKeys / 8];
  uint32_t bits[kQWaves][kQMaxWords];
  bf16_t qrows[32][D];                  // raw_q rows of the tile's queries
};

// Orders one wave's LDS accesses across its lanes (arrays private to a wave).
TAO_DEV void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
  constexpr int G = 8;                           // coarse_group (checked at launch)
  const int epoch = p.first_epoch + erel;
  const int K = epoch / G, pending = epoch % G;
  const int E = G * coarse + pending;
  const int words = (epoch + 31) >> 5;
  const bf16_t* pw_g = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
  const SwRows sw_g{p.sw + (size_t)bh * p.fine_cap * D,
                    p.psw_pool + ((size_t)erel * BH + bh) * 8 * D, K * G};
  for (int i = threadIdx.x; i < nq * (D / 8); i += kQThreads) {
    const int r = i / (D / 8), c = i % (D / 8);
    *(uint4*)&sm.qrows[r][c * 8] =
        *(const uint4*)(p.rq + b * p.rq_sb + (int64_t)(q_first + r) * p.rq_st + h * p.rq_sh + c * 8);
  }
  __syncthreads();
  const bf16_t* pw = pw_g;
  const SwRows swr = sw_g;
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
  for (int qi = w; qi < nq; qi += kQWaves) {
    const int t = q_first + qi;
    query_weights<D>(sm.qrows[qi], lane, hw);
    for (int i = lane; i < words; i += 64) bits[i] = 0u;
    wave_sync();
    // ---- page masses of the completed pages, stable top-`coarse`, ascending
    if (coarse > 0) {
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
      wave_sync();
      int placed = 0;
      for (int c0 = 0; c0 < K; c0 += 64) {
        const int i = c0 + lane;
        const bool pick = i < K && key_rank(keys, K, keys[i]) < coarse;
        const unsigned long long ball = __ballot(pick);
        if (pick) chosen[placed + __popcll(ball & ((1ull << lane) - 1ull))] = i;
        placed += __popcll(ball);
      }
      wave_sync();
    }
    // ---- candidate masses: 8 fines of each chosen page, then the pending fines
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
    wave_sync();
    // ---- stable top-M candidates -> bitmask
    for (int j = lane; j < E; j += 64)
      if (key_rank(keys, E, keys[j]) < M) {
        int page, id;
        cand(j, page, id);
        atomicOr(&bits[id >> 5], 1u << (id & 31));
      }
    wave_sync();
    uint32_t* dst = p.qsel + ((size_t)(b * p.T + t) * p.H + h) * p.qsel_words;
    for (int i = lane; i < words; i += 64) dst[i] = bits[i];
    wave_sync();                                 // h, keys and bits are reused
  }
}

// ---------------------------------------------------------------------------
// Per-query routes, lane per (query, row) pair: the same arithmetic as
// route_queries_kernel with the channel sum of one mass done by one lane in
// registers, in the fold order (pairs (e, e + 64) for D = 128, then
// (e, e + 32), (e, e + 16), ..., (e, e + 1)), so no cross-lane reduction is
// needed. One 256-thread workgroup per (read tile of <= 32 queries, batch,
// head); the tile's h rows, page-weight rows and the segment-weight rows of
// its visible fines sit in LDS, and the (query, page) and (query, candidate)
// pairs are spread over all lanes. Keys are 32-bit: monotone bf16 score in
// the high half, 0xFFFF - index in the low half (same order as score_key).
constexpr int kTileQ = 32;

template <int D, int ROWS_ = (D == 64 ? 128 : 64)>
struct RouteTileGeo {
  static constexpr int PAD = D + 8;                  // padded LDS row (bf16)
  static constexpr int ROWS = ROWS_;                 // staged pw + sw rows
  static constexpr int KEYS = ROWS;                  // >= pages, >= candidates
  static constexpr int WORDS = ROWS / 32;
};
// Staged rows of the turn-route kernel (prefill turns reach further epochs).
template <int D>
constexpr int kTurnRows = D == 64 ? 256 : 160;

template <int D, int ROWS_ = (D == 64 ? 128 : 64)>
struct RouteTileSmem {
  using G = RouteTileGeo<D, ROWS_>;
  bf16_t h[kTileQ][G::PAD];
  bf16_t rows[G::ROWS][G::PAD];
  uint32_t keys[kTileQ][G::KEYS];
  uint8_t chosen[kTileQ][G::KEYS / 8];
  uint32_t bits[kTileQ][G::WORDS];
  float hf[4][D];                                    // one query's h per wave (fp32)
};

TAO_DEV uint32_t score_key32(float score_bf, int index) {
  bf16_t bits = f2bf(score_bf);
  if (bits == 0x8000) bits = 0;                      // -0 ties with +0, as in torch's sort
  return (bf16_order_key(bits) << 16) | (uint32_t)(0xFFFF - index);
}

TAO_DEV void unpack8(const uint4& u, float out[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

// r(fold_e r(r(h[e] * pw[e]) * sw[e])) (WITH_SW) or r(fold_e r(h[e] * pw[e])).
template <int D, bool WITH_SW>
TAO_DEV float lane_mass(const bf16_t* hrow, const bf16_t* pwrow, const bf16_t* swrow) {
  float s1[32];
#pragma unroll
  for (int c = 0; c < 4; ++c) {            // s1[8c + k], k < 8
    float part[D / 32][8];
#pragma unroll
    for (int b = 0; b < D / 32; ++b) {     // channels 8c + k + 32 b
      const int e0 = 8 * c + 32 * b;
      float hv[8], pv[8];
      unpack8(*(const uint4*)(hrow + e0), hv);
      unpack8(*(const uint4*)(pwrow + e0), pv);
      float sv[8];
      if constexpr (WITH_SW) unpack8(*(const uint4*)(swrow + e0), sv);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float x = rbf(hv[k] * pv[k]);
        part[b][k] = WITH_SW ? rbf(x * sv[k]) : x;
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if constexpr (D == 64)
        s1[8 * c + k] = part[0][k] + part[1][k];
      else
        s1[8 * c + k] = (part[0][k] + part[2][k]) + (part[1][k] + part[3][k]);
    }
  }
#pragma unroll
  for (int w = 16; w >= 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w; ++i) s1[i] += s1[i + w];
  return rbf(s1[0]);
}

// Lane-per-pair routing of nq queries whose h rows (sm.h) and page-weight /
// segment-weight rows (sm.rows: P page rows, then one row per fine id) are
// staged: coarse pages by page mass (stable top-`coarse`, then ascending, in
// sm.chosen), candidate masses, stable top-M; emit(q, rank, id) for every
// selected candidate (rank = position in score order). All threads call it.
template <int D, class SM, class Emit>
TAO_DEV void route_core(SM& sm, int nq, int K, int coarse, int E, int M, int P, int tid,
                        Emit emit) {
  constexpr int G = 8;
  // ---- coarse pages: stable top-`coarse` by page mass, listed ascending
  if (coarse >= K) {
    for (int i = tid; i < nq * K; i += kQThreads) sm.chosen[i / K][i % K] = (uint8_t)(i % K);
  } else {
    for (int i = tid; i < nq * K; i += kQThreads) {
      const int q = i / K, pg = i % K;
      const float m = lane_mass<D, false>(sm.h[q], sm.rows[pg], nullptr);
      sm.keys[q][pg] = score_key32(m, pg);
    }
    __syncthreads();
    // chosen flag in the low byte of the key slot's spare: rank < coarse
    for (int i = tid; i < nq * K; i += kQThreads) {
      const int q = i / K, pg = i % K;
      const uint32_t mine = sm.keys[q][pg];
      int rank = 0;
      for (int j = 0; j < K; ++j) rank += sm.keys[q][j] > mine;
      if (rank < coarse) {
        // ascending position = chosen pages with a smaller index
        int pos = 0;
        for (int j = 0; j < pg; ++j) {
          const uint32_t other = sm.keys[q][j];
          int r2 = 0;
          for (int l = 0; l < K; ++l) r2 += sm.keys[q][l] > other;
          pos += r2 < coarse;
        }
        sm.chosen[q][pos] = (uint8_t)pg;
      }
    }
  }
  __syncthreads();
  // ---- candidate masses: 8 fines of each chosen page, then the pending fines
  auto cand = [&](int q, int j, int& page, int& id) __attribute__((always_inline)) {
    if (j < G * coarse) {
      page = sm.chosen[q][j / G];
      id = page * G + j % G;
    } else {
      page = K;
      id = K * G + (j - G * coarse);
    }
  };
  for (int i = tid; i < nq * E; i += kQThreads) {
    const int q = i / E, j = i % E;
    int page, id;
    cand(q, j, page, id);
    const float m = lane_mass<D, true>(sm.h[q], sm.rows[page], sm.rows[P + id]);
    sm.keys[q][j] = score_key32(m, j);
  }
  __syncthreads();
  // ---- stable top-M per query -> bitmask
  for (int i = tid; i < nq * E; i += kQThreads) {
    const int q = i / E, j = i % E;
    const uint32_t mine = sm.keys[q][j];
    int rank = 0;
    for (int l = 0; l < E; ++l) rank += sm.keys[q][l] > mine;
    if (rank < M) {
      int page, id;
      cand(q, j, page, id);
      emit(q, rank, id);
    }
  }
}

template <int D>
__global__ __launch_bounds__(kQThreads) void route_tile_kernel(QueryRouteParams p) {
  using Geo = RouteTileGeo<D>;
  __shared__ RouteTileSmem<D> sm;
  constexpr int G = 8;                           // coarse_group (checked at launch)
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int b = bh / p.H, h = bh % p.H;
  // Tiles in reverse order: the latest tiles score the most keys.
  const int64_t* desc = p.tiles + 8 * ((int)gridDim.x / BH - 1 - (int)blockIdx.x / BH);
  if (!desc[6]) return;                          // no history: workgroup-uniform
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int q_first = (int)desc[0], nq = (int)desc[1];
  const int coarse = (int)desc[2], M = (int)desc[3], erel = (int)desc[4];
  const int epoch = p.first_epoch + erel;
  const int K = epoch / G, pending = epoch % G;
  const int E = G * coarse + pending;
  const int P = K + (pending > 0);
  const int words = (epoch + 31) >> 5;
  const bf16_t* pw_g = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
  const SwRows sw_g{p.sw + (size_t)bh * p.fine_cap * D,
                    p.psw_pool + ((size_t)erel * BH + bh) * 8 * D, K * G};
  // ---- stage: rows [0, P) page weights, [P, P + epoch) segment weights
  for (int i = tid; i < (P + epoch) * (D / 8); i += kQThreads) {
    const int r = i / (D / 8), c = i % (D / 8);
    const bf16_t* src = r < P ? pw_g + (size_t)r * D : sw_g.row(r - P, D);
    *(uint4*)&sm.rows[r][c * 8] = *(const uint4*)(src + c * 8);
  }
  for (int i = tid; i < kTileQ * Geo::WORDS; i += kQThreads) (&sm.bits[0][0])[i] = 0u;
  // ---- h of each query: wave w does queries w, w + 4, ...
  for (int qi = w; qi < nq; qi += 4) {
    query_weights<D>(p.rq + b * p.rq_sb + (int64_t)(q_first + qi) * p.rq_st + h * p.rq_sh,
                     lane, sm.hf[w]);
    wave_sync();
    for (int e = lane; e < D; e += 64) sm.h[qi][e] = f2bf(sm.hf[w][e]);
    wave_sync();
  }
  __syncthreads();
  route_core<D>(sm, nq, K, coarse, E, M, P, tid,
                [&](int q, int rank, int id) { atomicOr(&sm.bits[q][id >> 5], 1u << (id & 31)); });
  __syncthreads();
  for (int i = tid; i < nq * words; i += kQThreads) {
    const int q = i / words, wd = i % words;
    p.qsel[((size_t)(b * p.T + q_first + q) * p.H + h) * p.qsel_words + wd] = sm.bits[q][wd];
  }
}

// Turn routes of a prefill (route_kernel's turn mode) with the lane-per-pair
// core: one 256-thread workgroup per (16 consecutive turns, batch, head).
// The turns are split into runs that share a seal epoch (a run holds at most
// the turns of one epoch, within the tile's 32 queries); each run stages its
// epoch's rows once and routes its anchors together. Outputs as route_kernel: ids in score order into the turn's
// sel_pool slot; the publishing turn also writes the state's route, chosen
// pages and route size.
constexpr int kTurnGroup = 16;

template <int D>
__global__ __launch_bounds__(kQThreads) void route_turns_kernel(RouteParams p) {
  constexpr int ROWS = kTurnRows<D>;
  __shared__ RouteTileSmem<D, ROWS> sm;
  constexpr int G = 8;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int b = bh / p.H, h = bh % p.H;
  // Turn groups in reverse order: the latest turns score the most rows.
  const int t0 = ((p.n_turns + kTurnGroup - 1) / kTurnGroup - 1 - (int)blockIdx.x / BH) * kTurnGroup;
  const int t1 = min(p.n_turns, t0 + kTurnGroup);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int s0 = t0; s0 < t1;) {
    const int64_t* d0 = p.turns + 8 * s0;
    int s1 = s0 + 1;
    while (s1 < t1 && p.turns[8 * s1 + 1] == d0[1]) ++s1;
    const int erel = (int)d0[1], K = (int)d0[2], pending = (int)d0[3];
    const int coarse = (int)d0[4], M = (int)d0[5];
    const int epoch = K * G + pending, P = K + (pending > 0), E = G * coarse + pending;
    const int nq = s1 - s0;
    const bf16_t* pw_g = p.pw_pool + ((size_t)erel * BH + bh) * p.pool_pcap * D;
    const SwRows sw_g{p.sw + (size_t)bh * p.fine_cap * D,
                      p.psw_pool + ((size_t)erel * BH + bh) * 8 * D, K * G};
    __syncthreads();                               // the previous run is done with sm
    for (int i = tid; i < (P + epoch) * (D / 8); i += kQThreads) {
      const int r = i / (D / 8), c = i % (D / 8);
      const bf16_t* src = r < P ? pw_g + (size_t)r * D : sw_g.row(r - P, D);
      *(uint4*)&sm.rows[r][c * 8] = *(const uint4*)(src + c * 8);
    }
    for (int qi = w; qi < nq; qi += 4) {
      const int64_t anchor = p.turns[8 * (s0 + qi)];
      query_weights<D>(p.rq + b * p.rq_sb + anchor * p.rq_st + h * p.rq_sh, lane, sm.hf[w]);
      wave_sync();
      for (int e = lane; e < D; e += 64) sm.h[qi][e] = f2bf(sm.hf[w][e]);
      wave_sync();
    }
    __syncthreads();
    route_core<D>(sm, nq, K, coarse, E, M, P, tid, [&](int q, int rank, int id) {
      const int64_t* dq = p.turns + 8 * (s0 + q);
      p.sel_pool[((size_t)dq[6] * BH + bh) * p.sel_cap + rank] = id;
      if (dq[7]) p.sel[(size_t)bh * p.sel_cap + rank] = id;
    });
    for (int q = 0; q < nq; ++q) {
      if (!p.turns[8 * (s0 + q) + 7]) continue;   // workgroup-uniform
      for (int i = tid; i < coarse; i += kQThreads)
        p.chosen[(size_t)bh * p.chosen_cap + i] = sm.chosen[q][i];
      if (bh == 0 && tid == 0) p.header[1] = M;
    }
    s0 = s1;
  }
}

}  // namespace

hipError_t launch_route_queries(const QueryRouteParams& p, int head_dim, hipStream_t s) {
  if (p.n_tiles <= 0) return hipSuccess;
  if (p.qsel_words < 1 || p.qsel_words > kQMaxWords || p.group != 8 || p.max_epoch < 1)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)(p.n_tiles * p.B * p.H));
  // Lane-per-pair kernel when every tile's page and fine rows fit its LDS
  // rows (and tiles hold <= 32 queries); else one wave per query.
  const int rows = p.max_epoch / p.group + 1 + p.max_epoch;
  if (head_dim == 128) {
    if (rows <= RouteTileGeo<128>::ROWS)
      hipLaunchKernelGGL(route_tile_kernel<128>, grid, dim3(kQThreads), 0, s, p);
    else
      hipLaunchKernelGGL(route_queries_kernel<128>, grid, dim3(kQThreads), 0, s, p);
  } else if (head_dim == 64) {
    if (rows <= RouteTileGeo<64>::ROWS)
      hipLaunchKernelGGL(route_tile_kernel<64>, grid, dim3(kQThreads), 0, s, p);
    else
      hipLaunchKernelGGL(route_queries_kernel<64>, grid, dim3(kQThreads), 0, s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_route(const RouteParams& p, int head_dim, hipStream_t s) {
  if (p.completed > kMaxSort || p.group * p.coarse + p.pending > kMaxSort)
    return hipErrorInvalidValue;
  // Turn mode: the lane-per-pair kernel when every turn's rows fit its LDS.
  if (p.turns && p.gate.header) return hipErrorInvalidValue;   // gates serve single turns
  if (p.turns && p.n_turns > 0 && p.group == 8 && p.max_epoch >= 1 &&
      p.max_epoch / 8 + 1 + p.max_epoch <= (head_dim == 64 ? kTurnRows<64> : kTurnRows<128>)) {
    const dim3 tgrid((unsigned)(p.B * p.H * ((p.n_turns + kTurnGroup - 1) / kTurnGroup)));
    if (head_dim == 128)
      hipLaunchKernelGGL(route_turns_kernel<128>, tgrid, dim3(kQThreads), 0, s, p);
    else if (head_dim == 64)
      hipLaunchKernelGGL(route_turns_kernel<64>, tgrid, dim3(kQThreads), 0, s, p);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  }
  // Single turn (a stream's refresh): the LDS-staged kernel when its rows fit.
  const int pages = p.completed + (p.pending > 0 ? 1 : 0);
  if (!p.turns && pages <= kRefreshPages && p.group * p.coarse + p.pending <= kRefreshRows &&
      p.group == 8) {
    const dim3 rgrid((unsigned)(p.B * p.H));
    if (head_dim == 128)
      hipLaunchKernelGGL(route_refresh_kernel<128>, rgrid, dim3(kRefreshThreads), 0, s, p);
    else if (head_dim == 64)
      hipLaunchKernelGGL(route_refresh_kernel<64>, rgrid, dim3(kRefreshThreads), 0, s, p);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  }
  const dim3 grid((unsigned)(p.B * p.H * (p.turns ? p.n_turns : 1)));
  if (head_dim == 128)
    hipLaunchKernelGGL(route_kernel<128>, grid, dim3(kRouteThreads), 0, s, p);
  else if (head_dim == 64)
    hipLaunchKernelGGL(route_kernel<64>, grid, dim3(kRouteThreads), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// The refresh and its fold in one launch when the route fits the staged
// refresh (single turn, group 8, rows within kRefreshPages / kRefreshRows);
// returns hipErrorNotSupported otherwise (the caller launches the two).
hipError_t launch_refresh_fold(const RouteParams& p, const FoldParams& f, int head_dim,
                               hipStream_t s) {
  const int pages = p.completed + (p.pending > 0 ? 1 : 0);
  if (p.turns || pages > kRefreshPages || p.group * p.coarse + p.pending > kRefreshRows ||
      p.group != 8 || f.group != 8 || p.selected != f.M || p.selected <= 0)
    return hipErrorNotSupported;
  if (head_dim == 128) {
    constexpr int CHUNKS = 128 / (kRefreshThreads / 64);
    hipLaunchKernelGGL(refresh_fold_kernel<128>, dim3((unsigned)(p.B * p.H * CHUNKS)),
                       dim3(kRefreshThreads), 0, s, p, f);
  } else if (head_dim == 64) {
    constexpr int CHUNKS = 64 / (kRefreshThreads / 32);
    hipLaunchKernelGGL(refresh_fold_kernel<64>, dim3((unsigned)(p.B * p.H * CHUNKS)),
                       dim3(kRefreshThreads), 0, s, p, f);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace tao
