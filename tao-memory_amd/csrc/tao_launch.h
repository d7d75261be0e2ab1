// Internal launch interface between the C-ABI layer (abi.hip) and the
// kernel translation units. Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tao_memory.h"
#include "tao_common.h"

namespace tao {

// Record a message for tao_last_error() (thread-local).
void set_error(const char* msg);

constexpr int kThreads = 256;   // 4 wave64 per workgroup
constexpr int kMaxWindow = 768;   // serve_limit = local_keep + fine_tokens
constexpr int kStepRec = 4;       // header floats of one decode record
#ifndef TAO_LOCAL_KEY_DIV
#define TAO_LOCAL_KEY_DIV 2
#endif
constexpr int kLocalKeyDiv = TAO_LOCAL_KEY_DIV;   // keys per local workgroup = D / div
constexpr int kFineRows = 32;     // rows of the folded route per fine-read workgroup

// Keys per local-attention workgroup: D / kLocalKeyDiv, at least one load
// pass of the workgroup (kThreads / (D / 8) rows).
__host__ __device__ constexpr int local_keys(int head_dim) {
  return head_dim / kLocalKeyDiv > 256 / (head_dim / 8) ? head_dim / kLocalKeyDiv
                                                         : 256 / (head_dim / 8);
}

// Local-attention workgroups per (batch, head).
__host__ __device__ constexpr int local_units(int head_dim) {
  return (kMaxWindow + local_keys(head_dim) - 1) / local_keys(head_dim);
}

// Fine-read workgroups per (batch, head).
__host__ __device__ constexpr int fine_units(int head_dim) { return head_dim / kFineRows; }

// Per (batch, head) decode scratch, in floats: local_units(D) local-attention
// records, one fine record (den in the header, num[D]), one coarse record
// (coarse[D]) and three fusion-weight records (the local, coarse and fine
// branch weights of every channel), each of (kStepRec + D) floats.
__host__ __device__ inline size_t step_floats(int head_dim, int sel_cap) {
  (void)sel_cap;
  return (size_t)(local_units(head_dim) + 5) * (head_dim + kStepRec);
}

// Workspace layout (bytes from the start of tao_state_dev::workspace):
//   [0, count_off)        fp32 decode scratch [B*H][step_floats(D, sel_cap)]
//   [count_off, plan_off) uint32 arrival counters of the decode step: one per
//                         (batch, head), then one for the launch, each on
//                         its own 128-byte line (zero between steps)
//   [plan_off, total)     int64 prefill plan (plan_words)
struct WorkspaceLayout {
  size_t parts_off, count_off, plan_off, plan_words, total;
};

// Decode-step arrival counters for B*H heads, one per 128-byte line (the
// heads' atomics never share a cache line): counter i at word
// i * kCounterStride.
constexpr int kCounterStride = 32;
__host__ __device__ inline size_t step_counters(int batch, int heads) {
  return (size_t)batch * heads + 1;
}

WorkspaceLayout workspace_layout(int batch, int heads, int head_dim, int sel_cap,
                                 int plan_words);

// Per-tensor [B, T, H, D] view in elements.
struct TokView {
  const bf16_t* p;
  int64_t sb, st, sh;
};

struct DecodeParams {
  TokView q, k, v, rq, rk;
  bf16_t* ring_k; bf16_t* ring_v; bf16_t* ring_raw;
  const bf16_t* bank; const bf16_t* sw; const bf16_t* pw;
  const int32_t* sel;
  int64_t* header;
  const void* fa; const void* fb; int f_dtype;
  int64_t fa_s[3], fb_s[3];
  float gain;
  bf16_t* out; int64_t out_sb, out_sh;
  float* parts;
  unsigned* counters;   // step_counters(B, H) arrival counters, kCounterStride apart
                        // (zero between steps)
  const float* fold_g; const float* fold_den;   // folded route (G^T, den weights)
  const float* coarse_g;   // folded coarse read (G^T), read when coarse_on
  long long pos_hint;   // cursor of this step, or -1: read header[0]
  int B, H, keep, fine, group, fine_cap, page_cap, sel_cap;
  int coarse_on;
  int win_n_old, win_first;   // the window at pos_hint (set by launch_decode_step)
  unsigned long long* stamps;   // diagnostic clock stamps of this launch (null: none;
                                // set by launch_decode_step while a recorder is on)
};

// Words per workgroup of a decode step's stamp frame: the 100 MHz device
// clock (s_memrealtime) at entry, after the loads of a local unit landed
// (its scores), after the unit's record stores issued, after they were
// acknowledged (the release barrier), after the arrival count, after the
// merge (the head's last arrival only, else 0); then the unit's identity
// (j << 32 | batch * H + head) and its placement (XCC << 32 | __smid()).
constexpr int kStampWords = 8;

// Diagnostic stamp recorder of eager decode steps (single-threaded use):
// launch i with a host cursor writes frame i % frames of buf (frame_words
// words each, at least grid * kStampWords). A null buf stops it.
int step_stamps_set(void* buf, long long frames, long long frame_words);
long long step_stamps_count();

// M = selected fines of the current route (0 before the first seal: no
// fine read). The fine read uses the folded route (launch_fold); with
// coarse_on the step also reads the folded coarse matrix (launch_coarse_fold).
hipError_t launch_decode_step(const DecodeParams& p, int head_dim, int M, hipStream_t s);

// Batched decode step over R requests of one layer (each state batch 1):
// per-request buffers in a device table; cursor and route size read from
// each request's header[0] / header[1].
struct BatchReq {
  bf16_t* ring_k; bf16_t* ring_v; bf16_t* ring_raw;
  const float* fold_g; const float* fold_den; const float* coarse_g;   // coarse_g may be null
  int64_t* header;
  float* parts;
};

struct BatchStepParams {
  TokView q, k, v, rq, rk;       // [R, 1, H, D]: request r = batch row r
  const void* fa; const void* fb; int f_dtype;
  int64_t fa_s[3], fb_s[3];
  float gain;
  bf16_t* out; int64_t out_sb, out_sh;
  const BatchReq* table;
  int R, H, keep, fine, group;
  int coarse_values;             // the states carry the coarse value branch
};
hipError_t launch_batch_step(const BatchStepParams& p, int head_dim, hipStream_t s);

// Route refresh gated on the device cursor, for a decode step captured in a
// graph and replayed for later tokens: a kernel given a gate with a header
// reads the cursor header[0] (the position of the token about to be
// decoded) and exits at once unless it is a refresh turn of the stream's
// layer: limit, or first + k * period for k >= 0 (the stagger of
// tao_stream.py:202-208). Without a header the kernel always runs.
struct TurnGate {
  const int64_t* header;
  long long first, period, limit;
};

__device__ inline bool gate_closed(const TurnGate& g) {
  if (!g.header) return false;
  const long long pos = g.header[0];
  return !(pos == g.limit || (pos >= g.first && (pos - g.first) % g.period == 0));
}

struct FoldParams {
  const bf16_t* bank; const bf16_t* sw; const bf16_t* pw;
  const int32_t* sel;
  float* fold_g; float* fold_den;
  int B, H, group, fine_cap, page_cap, sel_cap, M;
  TurnGate gate;
};
hipError_t launch_fold(const FoldParams& p, int head_dim, hipStream_t s);

// Page value matrices of completed pages [first_page, first_page + count):
// page_c[g][e][d] = r(sum_s sw[8g + s][d] * C^T_{8g+s}[e][d]).
struct PageCoarseParams {
  const bf16_t* bank; const bf16_t* sw; bf16_t* page_c;
  int B, H, fine_cap, page_cap, group, first_page, count;
};
hipError_t launch_page_coarse(const PageCoarseParams& p, int head_dim, hipStream_t s);

// Folded coarse reads G^T(n)[e][d] = sum_{p < n} softmax_p(page_z)[d] *
// page_c[p][e][d] for n in [n_first, n_first + n_count), one pass over the
// pages; output n_first + i goes to out + i * B*H*D*D as fp32 (out_f32) or
// bf16.
struct CoarseFoldParams {
  const bf16_t* page_z; const bf16_t* page_c;
  void* out; int out_f32;
  int B, H, page_cap, n_first, n_count;
};
hipError_t launch_coarse_fold(const CoarseFoldParams& p, int head_dim, hipStream_t s);

// tao_decode_step with the step's cursor given by the caller (position >= 0)
// instead of read from header[0] on the device; used by the stream driver.
// records / counters: the step's per-head records (B * H * step_floats(D)
// floats) and its step_counters(B, H) arrival counters, or both null for the
// state's workspace (then required).
int decode_step_at(const tao_state_dev* st, const tao_tokens* tok, const tao_fusion* fu,
                   int32_t selected, void* out, const int64_t* out_s, void* stream,
                   long long position, float* records = nullptr,
                   unsigned* counters = nullptr);

// tao_route / tao_fold_route with a turn gate (TurnGate{} = ungated).
int route_at(const tao_state_dev* st, const void* raw_q_row, const int64_t* rq_s,
             int32_t completed, int32_t pending, int32_t coarse, int32_t selected,
             const TurnGate& gate, void* stream);
int fold_at(const tao_state_dev* st, int32_t selected, const TurnGate& gate, void* stream);
// route_at then fold_at of the same route, as one launch where the route
// fits the fused kernel (launch_refresh_fold).
int refresh_fold_at(const tao_state_dev* st, const void* raw_q_row, const int64_t* rq_s,
                    int32_t completed, int32_t pending, int32_t coarse, int32_t selected,
                    const TurnGate& gate, void* stream);

// The decode step's kernel arguments for a state, fusion and output buffer,
// recorded once (decode_record) and dispatched per token with that token's
// operands and cursor patched in (decode_replay).
int decode_record(const tao_state_dev* st, const tao_tokens* tok, const tao_fusion* fu,
                  int32_t selected, void* out, const int64_t* out_s, DecodeParams* rec);
int decode_replay(const DecodeParams& rec, const tao_tokens* tok, int head_dim,
                  int32_t selected, long long position, void* stream);

// fp32 full-sequence read (full_f32.hip): operand views in fp32 elements,
// the call's workspace carved by f32_layout.
struct F32View {
  const float* p;
  int64_t sb, st, sh;
};

struct F32Params {
  F32View q, k, v, rq, rk;
  const void* fa; const void* fb; int f_dtype;
  int64_t fa_s[3], fb_s[3];
  float gain;
  float* out; int64_t out_sb, out_st, out_sh;
  float* local;    // [B, T, H, D]
  float* fine_z;   // [B, H, S, D]
  float* bank;     // [B, H, S, D, D], C[d][e]
  float* pz;       // [B, H, P8, 8, D]: logsumexp of each page's first n fines
  float* swt;      // [B, H, P8, 36, D]: segment weights under each prefix
  float* pc;       // [B, H, Pc, D, D] completed pages' value matrices, or null
  int32_t* sel_out;   // optional [B, T, H, sel_cap] selections (score order, -1 pad)
  int sel_cap;
  tao_stream_cfg cfg;
  int B, H, D, T, S, P8, Pc, coarse_values;
};
size_t f32_workspace_floats(int B, int H, int D, int64_t T, int coarse_values);
int f32_layout(F32Params& p, float* ws, int64_t T, int coarse_values);
// 1 when T fits the read kernel's LDS tables (pages, candidates, selections).
int f32_limits(const tao_stream_cfg& cfg, int64_t T, int64_t* pages, int64_t* cand);
// own_local: run the fp32 local attention into p.local first (else the
// caller's local attention output is there).
hipError_t launch_full_f32(const F32Params& p, hipStream_t s, bool own_local);

struct AppendParams {
  TokView k, v, rk;
  bf16_t* ring_k; bf16_t* ring_v; bf16_t* ring_raw;
  int B, H, D, L, first, count;
  int64_t pos;
};
hipError_t launch_ring_append(const AppendParams& p, hipStream_t s);

// One route refresh. Single-turn mode (turns == nullptr) routes the anchor
// row rq against the state's current epoch. Turn mode: workgroup
// (turn, b, h) reads turns[turn * 8 + ...] = {anchor token, epoch, completed,
// pending, coarse, selected, output slot, write_state} and takes its page
// weights and pending-fine segment weights from the epoch pools.
struct RouteParams {
  const bf16_t* rq; int64_t rq_sb, rq_st, rq_sh;
  const bf16_t* pw; const bf16_t* sw;
  const bf16_t* pw_pool; const bf16_t* psw_pool; int pool_pcap;
  int32_t* sel; int32_t* chosen; int64_t* header;
  int32_t* sel_pool;
  const int64_t* turns; int n_turns;
  int B, H, fine_cap, page_cap, sel_cap, chosen_cap, group;
  int completed, pending, coarse, selected;
  int max_epoch;                 // turn mode: largest epoch of any turn (0: unknown)
  TurnGate gate;                 // single-turn mode only
};
hipError_t launch_route(const RouteParams& p, int head_dim, hipStream_t s);
// A single-turn route refresh and its fold in one launch (both parameter
// sets describe the same state and route size); hipErrorNotSupported when
// the route does not fit the fused kernel.
hipError_t launch_refresh_fold(const RouteParams& p, const FoldParams& f, int head_dim,
                               hipStream_t s);

// Per-query routes of the full-sequence read: every history query of a read
// tile routes itself against its tile's epoch; selections are bitmasks
// qsel[((b * T + t) * H + h) * qsel_words + word].
struct QueryRouteParams {
  const bf16_t* rq; int64_t rq_sb, rq_st, rq_sh;
  const bf16_t* sw;
  const bf16_t* pw_pool; const bf16_t* psw_pool; int pool_pcap;
  const int64_t* tiles; int n_tiles;
  uint32_t* qsel; int qsel_words;
  int first_epoch, max_epoch;      // max_epoch: largest epoch of any read tile
  int B, H, T, group, fine_cap;
};
hipError_t launch_route_queries(const QueryRouteParams& p, int head_dim, hipStream_t s);
constexpr int kQueryRouteMaxKeys = 512;   // pages or candidates of one query route

struct WriterParams {
  TokView rk, v;                 // token operands (positions >= new_base)
  const bf16_t* ring_raw; const bf16_t* ring_v;
  bf16_t* bank; bf16_t* fine_z;
  const int64_t* starts;         // device [count] absolute start positions
  int64_t new_base;
  int B, H, L, fine_cap, first_slot, count;
  int z_only;                    // write fine_z only (the caller owns the C slots)
};
hipError_t launch_writer(const WriterParams& p, int head_dim, hipStream_t s);

// fine_mass (feature writers): a page's z is r(log) of its run's fp32 mass
// total at the page's last fine (see FeatureDescParams) instead of
// r(logsumexp) of its fines' z.
struct EpilogueParams {
  const bf16_t* fine_z; bf16_t* fine_sw; bf16_t* page_z; bf16_t* page_w;
  const float* fine_mass;
  int B, H, fine_cap, page_cap, group, slot, pages;
  int recompute;                 // 0: keep page_z[slot's group] (snapshot import)
};
hipError_t launch_seal_epilogue(const EpilogueParams& p, int head_dim, hipStream_t s);

struct AttnParams {
  TokView q, k, v;
  const bf16_t* ring_k; const bf16_t* ring_v;
  bf16_t* out;                   // [B, T, H, D] contiguous (T = query rows)
  const int64_t* tiles;          // device [n_tiles][3]: first q row, count, key_start
  int64_t qpos0;                 // absolute position of query row 0
  int64_t kpos0;                 // absolute position of key row 0 (older keys: ring)
  int B, H, L, T, n_tiles;
  float* lse;                    // optional [B, T, H]: log2-sum-exp of the scaled scores
};
hipError_t launch_local_attention(const AttnParams& p, int head_dim, hipStream_t s);

// Completed pages of a prefill call: page descriptors and final segment
// weights of pages [first_page, first_page + count).
struct PagesParams {
  const bf16_t* fine_z; bf16_t* fine_sw; bf16_t* page_z;
  const float* fine_mass;        // feature writers (see EpilogueParams)
  int B, H, fine_cap, page_cap, group, first_page, count;
};
hipError_t launch_pages(const PagesParams& p, int head_dim, hipStream_t s);

// Seal epochs [first_epoch, first_epoch + count) of a prefill call (epoch =
// number of visible fines): pending summary, pending segment weights and
// page weights into the pools; the last epoch is also published to the state.
struct EpochParams {
  const bf16_t* fine_z; bf16_t* fine_sw; bf16_t* page_z; bf16_t* page_w;
  const float* fine_mass;        // feature writers (see EpilogueParams)
  bf16_t* pw_pool; bf16_t* psw_pool; int pool_pcap;
  int B, H, fine_cap, page_cap, group, first_epoch, count;
};
hipError_t launch_epochs(const EpochParams& p, int head_dim, hipStream_t s);

// MFMA selected read + fusion over query tiles (<= 32 queries sharing one
// route). tiles[t * 8 + ...] = {first query, count, route slot, selected,
// epoch, sw split, fine_on, completed pages}. With coarse_pool, tiles with
// completed >= 1 add the coarse read h . G^T(completed) from
// coarse_pool[completed - coarse_first].
struct ReadTilesParams {
  TokView rq;
  const bf16_t* bank; const bf16_t* sw;
  const bf16_t* pw_pool; const bf16_t* psw_pool; int pool_pcap;
  const int32_t* sel_pool;
  const bf16_t* local;           // [B, T, H, D] contiguous
  const void* fa; const void* fb; int f_dtype;
  int64_t fa_s[3], fb_s[3];
  float gain;
  bf16_t* out; int64_t out_sb, out_st, out_sh;
  const int64_t* tiles; int n_tiles;
  int B, H, T, group, fine_cap, sel_cap;
  const bf16_t* coarse_pool; int coarse_first;
  // Per-query selections (plans with query routes): bitmasks as written by
  // route_queries, the plan's first epoch; null for turn routes.
  const uint32_t* qsel; int qsel_words; int first_epoch;
  // Optional saves (null = skip): pre-fusion heads [B, T, H, D], denominators [B, T, H].
  bf16_t* save_coarse; bf16_t* save_fine; float* save_den;
  // Feature writers: the state's fine descriptors [B, H, fine_cap, D]; the
  // read is the numerator-only mixture. With page values (turn routes), the
  // coarse read mixes the completed pages of a tile's chunk from the state's
  // page descriptors and page matrices (C^T) in place of coarse_pool.
  const bf16_t* fine_z;
  const bf16_t* page_z; const bf16_t* page_c; int page_cap;
};
hipError_t launch_read_tiles(const ReadTilesParams& p, int head_dim, hipStream_t s);

// ---- full-sequence backward (train_bwd.hip)
// Fusion adjoint: from the upstream gradient and the forward's saves to the
// branch adjoints, the fusion's part of d raw_q, d fusion_a / d fusion_b
// (accumulated, zeroed by the caller), and the local attention's delta.
struct TrainBwdParams {
  const bf16_t* grad; int64_t g_sb, g_st, g_sh;
  TokView rq;
  const bf16_t* local; const bf16_t* coarse; const bf16_t* fine; const float* den;
  const void* fa; const void* fb; int f_dtype;
  int64_t fa_s[3], fb_s[3];
  float gain;
  int B, T, H, first_fine, first_coarse, coarse_values;
  bf16_t* dlocal; float* delta; float* dcoarse; float* dnum; float* dden; float* drq;
  float* dfa; float* dfb;
  bf16_t* h;                     // h = softmax(raw_q) [B, T, H, D]
  float* dalpha_parts;           // nullable: one d alpha partial per workgroup
  float* dalpha;                 // fp32 scalar: the sum of the partials
};
hipError_t launch_fuse_bwd(const TrainBwdParams& p, int head_dim, hipStream_t s);
int fuse_bwd_workgroups(int T, int B, int H);   // d alpha partials launch_fuse_bwd writes

// Local attention adjoints with the full-sequence windows (query q sees keys
// [max(0, ft * (q / ft) - keep), q]).
struct AttnBwdParams {
  TokView q, k, v;
  const bf16_t* dout;            // d local, bf16 [B, T, H, D] contiguous
  const float* lse; const float* delta;   // [B, T, H]
  bf16_t* dq; bf16_t* dk; float* dv;      // dv fp32 (the writer's part is added later)
  int B, H, T, ft, keep;
};
hipError_t launch_attn_bwd(const AttnBwdParams& p, int head_dim, hipStream_t s);

// Memory-branch adjoints: selected read, coarse read, page / segment
// softmaxes and logsumexps, the softmax writer, and the final d raw_q /
// d raw_k / dv. fp32 accumulators are zeroed by the caller: dsw_tile, dpw,
// dsw, dpz, dz, dc, dgc (dh is written in full).
struct MemBwdParams {
  const bf16_t* bank; const bf16_t* fine_sw; const bf16_t* page_z; const bf16_t* page_c;
  const bf16_t* pw_pool; const bf16_t* psw_pool; int pool_pcap;
  const bf16_t* coarse_pool; int coarse_first, coarse_count;
  const uint32_t* qsel; int qsel_words;
  TokView raw_k, v;
  const bf16_t* h; const float* dnum; const float* dden; const float* dcoarse;
  const float* drq_fuse;
  float* dh;                     // [B, T, H, D]
  float* dpw;                    // [n_tiles][B*H][pool_pcap][D]
  float* dsw_tile;               // [n_tiles][B*H][v_max][D]
  float* dgc;                    // [coarse_count][B*H][D][D]  (dG^T [e][d])
  float* dc;                     // [B*H][v_max][D][D]         (dC^T [e][d])
  float* dsw;                    // [B*H][v_max][D]
  float* dpz;                    // [B*H][page_cap][D]
  float* dz;                     // [B*H][v_max][D]
  float* dv;                     // [B, T, H, D] fp32 (local part in, writer part added)
  bf16_t* draw_q; bf16_t* draw_k; bf16_t* dv_out;
  int B, H, T, ft, keep, group, fine_cap, page_cap, v_max, coarse_values;
  // Value matrices not from the softmax writer (regularized writer): the
  // writer adjoint takes only the z path, and dk_extra (fp32 [B, T, H, D],
  // nullable) is added to d raw_k of the block tokens.
  int values_external;
  const float* dk_extra;
  // With values_external and page values: d page_c (C^T layout, fp32
  // [B*H][dpc_cap][D][D], zeroed by the caller) accumulates here.
  float* dpc; int dpc_cap;
};
// The memory branch in two parts: read_part (the read's adjoints down to dC
// and dz) and writer_part (the writer adjoint and the finish); a caller may
// change dC's consumers in between.
hipError_t launch_mem_bwd_read(const MemBwdParams& p, int head_dim, hipStream_t s);
hipError_t launch_mem_bwd_writer(const MemBwdParams& p, int head_dim, hipStream_t s);

// ---- non-preset fine writers and the channel-given selected read

// Simplex-feature statistics of N token blocks: k, v [N, T, H, D] bf16 with
// element strides (block, token, head). mode 0: gram, cross (+ mass if set);
// mode 1: gram receives square_mass [N, H, D], plus cross and mass.
struct WriterStatsParams {
  const bf16_t* k; const bf16_t* v;
  int64_t k_s[3], v_s[3];
  int N, T, H, mode;
  float* gram; float* cross; float* mass;
  // Ring mode (starts != null): block n = blk * B + b is the 256-token block
  // starting at absolute position starts[blk] of batch row b; rows at or
  // after new_base come from k / v (strides: batch, token, head), older rows
  // from the token ring (slot = position mod L).
  const int64_t* starts; int64_t new_base;
  const bf16_t* ring_raw; const bf16_t* ring_v;
  int L, B;
};
hipError_t launch_writer_stats(const WriterStatsParams& p, int head_dim, hipStream_t s);

struct AssocSolveParams {
  const float* gram; const float* cross;
  int count;
  bf16_t* out;            // [count, D, D] rows d, columns e
  int32_t* info;          // nullable [count]
  // to_slots 1: matrix (blk, b, h) = (mat / (B H), mat / H % B, mat % H)
  // goes transposed (C^T[e][d]) into slot first_slot + blk of out viewed as
  // [B, H, cap, D, D]; 2: the same for page first_slot + blk ... only blocks
  // whose fine slot (fine_first + blk) completes a page (slot % group ==
  // group - 1), into page slot / group.
  int to_slots, B, H, cap, first_slot, fine_first, group;
  // Optional (to_slots 0): the fp32 solution [count, D, D] (rows d) instead
  // of the bf16 one; and a right-hand side other than cross: matrix
  // mat = (blk * B + b) * H + h takes rhs_t[(b H + h) rhs_cap + blk] as
  // its transpose ([e][d], fp32).
  float* out_f32;
  const float* rhs_t; int rhs_cap;
};
hipError_t launch_association_solve(const AssocSolveParams& p, int head_dim, hipStream_t s);

// Regularized writer backward over the call's fine blocks (tao_train_backward;
// association_writer.py:11-32 differentiated): matrix mat = (f B + b) H + h
// belongs to tokens [ft f, ft f + ft) of batch row b, head h. With
// A = gram + tr(gram)/D I, Y = A^{-1} cross (the fp32 C) and W = A^{-1} dC:
//   S = dG + dG^T, dG = -W Y^T + tr(-W Y^T)/D I             (assoc_gram_bwd)
//   du = V W^T + U S, dv += U W, dk = p (du - sum_d p du)   (assoc_block_bwd)
// with u = r(p), p = softmax_D(raw_k) per token.
struct AssocBwdParams {
  const float* w; const float* y; float* s;   // [mats][D][D]
  TokView raw_k, v;
  float* dk;                     // [B, T, H, D] fp32, written for block tokens
  float* dv;                     // [B, T, H, D] fp32, accumulated
  int mats, B, H, T, ft;
  // Feature writers (nullable): d of the block's feature mass sum_t u_t
  // [mats][D], added to every token's du before the feature softmax.
  const float* dmass;
};
hipError_t launch_assoc_gram_bwd(const AssocBwdParams& p, int head_dim, hipStream_t s);
// Pages of the regularized writer: page_sum writes the in-order sums of each
// completed page's group fines' statistics (x: [fines * B][H][dd] in (f, b, h)
// order -> out [pages * B][H][dd]); page_to_fines adds a page's W and S to
// each of its fines' (w, s: [fines * B][H][D][D], page ones after them).
hipError_t launch_page_sum(const float* x, float* out, int pages, int group, int B, int H,
                           int64_t dd, hipStream_t s);
hipError_t launch_page_to_fines(float* w, float* s_, const float* wp, const float* sp, int fines,
                                int group, int B, int H, int64_t dd, hipStream_t s);
hipError_t launch_assoc_block_bwd(const AssocBwdParams& p, int head_dim, hipStream_t s);
// starts[i] = i * step (the token blocks of a full-sequence call).
hipError_t launch_block_starts(int64_t* starts, int count, int64_t step, hipStream_t s);

struct StructuredParams {
  const float* square; const float* cross; const float* mass;
  int count_mats;
  float count;            // token count behind the statistics
  bf16_t* out;
  // to_slots 1: matrix (blk, b, h) goes transposed into fine slot
  // first_slot + blk of out viewed as [B, H, cap, D, D] (as AssocSolveParams);
  // 2: only blocks whose slot completes a page, into page slot / group.
  int to_slots, B, H, cap, first_slot, group;
};
hipError_t launch_structured_matrix(const StructuredParams& p, int head_dim, hipStream_t s);

// ---- feature writers' read adjoint (mix_bwd.hip)
// The numerator-only mixture read of the full-sequence path
// (tao_stream.py:600-662 with feature_read_coefficients,
// association_writer.py:46-53): query q reads items m (its selected fines, or
// for the coarse read the completed pages of its tile) with
// mass_m = sum_d h[d] exp(z_m[d]), w_m = mass_m / sum_m' mass_m' and
// out[e] = sum_m sum_d r(w_m h[d]) C_m[d][e]. Given d out, with
// dch_m[d] = sum_e dout[e] C_m[d][e] and dw_m = sum_d dch_m[d] h[d]:
//   dC_m[d][e] += r(w_m h[d]) dout[e],
//   dmass_m = (dw_m - sum_m' w_m' dw_m') / sum_m' mass_m',
//   dh[d] += sum_m (w_m dch_m[d] + dmass_m exp(z_m[d])),
//   dz_m[d] += sum_q dmass_m h[d] exp(z_m[d]).
struct MixBwdParams {
  const bf16_t* h;        // [B, T, H, D] the read's query weights
  const float* dout;      // [B, T, H, D] d fine (or d coarse)
  const bf16_t* z;        // [B, H, cap, D] item descriptors (fine_z or page_z)
  const bf16_t* mats;     // [B, H, cap, D, D] item matrices, C^T (bank or page_c)
  int cap;
  const uint32_t* qsel; int qsel_words;   // fine items: selection words; null: pages
  float* dh;              // [B, T, H, D] accumulated
  float* wv; float* dmv;  // [B, T, H, R] per query and item rank: w_m and dmass_m
  int R;                  // <= kMixMaxRank
  float* dmat;            // [B*H][n_items][D][D] d C^T (written)
  float* dz;              // [B*H][n_items][D] d z (written)
  int n_items;            // visible fines, or completed pages
  int B, H, T, ft, keep, group;
  int first_query;        // first token with this read (first_fine or first_coarse)
};
constexpr int kMixMaxRank = 64;      // items one query reads
constexpr int kMixMaxItems = 512;    // fine ids a query block can select
hipError_t launch_mix_bwd(const MixBwdParams& p, int head_dim, hipStream_t s);

// d mass of the feature writers' fines [mats][D] in (fine, b, h) order:
// dz_f / mass_f (z = r(log mass)) plus, for fines of the first `pages`
// completed pages, the page descriptor's dpz_p / mass_p with mass_p the sum
// of its fines' masses. dz: [B*H][fines][D]; dpz: [B*H][pages][D];
// mass: [mats][D]; extra (nullable): a further d mass [mats][D] added.
hipError_t launch_mass_grad(const float* dz, const float* dpz, const float* mass,
                            const float* extra, float* dmass, int fines, int pages, int group,
                            int B, int H, int head_dim, hipStream_t s);

// Structured-Gram matrix adjoint (structured_writer.py:16-34 under
// autograd): for `count_mats` matrices in (blk, b, h) order, from d C^T
// ([e][d] per matrix) at the statistics (square [mats][D], cross
// [mats][D][D] rows d, mass [mats][D], token count) to d square, d cross
// [mats][d][e] and d mass.
struct StructuredBwdParams {
  const float* square; const float* cross; const float* mass;
  const float* dct;       // matrix (blk, b, h) at [(b * H + h) * dct_cap + blk]
  int dct_cap, B, H;
  int count_mats;
  float count;
  float* dsquare; float* dcross; float* dmass;
};
hipError_t launch_structured_bwd(const StructuredBwdParams& p, int head_dim, hipStream_t s);
// S = diag(2 dsquare) as [mats][D][D] (the block adjoint's U S term).
hipError_t launch_square_diag(const float* dsquare, float* s_, int mats, int head_dim,
                              hipStream_t st);
// Adds each completed page's [pages * B][H][n] adjoint to its group fines'
// ([fines * B][H][n], (fine, b, h) order).
hipError_t launch_page_add(float* fine, const float* page, int pages, int group, int B, int H,
                           int64_t n, hipStream_t s);

// Feature-writer descriptors of `count` seals: matrix (blk, b, h) of the
// mass scratch [count * B][H][D] gives fine slot first_slot + blk its
// z = r(log mass) (tao_stream.py:60-65) and fine_mass[slot] its run's fp32
// mass total through it, in seal order. A run restarts at fine 0 and, with
// page_runs, at each page's first fine (slot % group == 0).
struct FeatureDescParams {
  const float* mass;
  bf16_t* fine_z; float* fine_mass;
  int count, B, H, cap, first_slot, group, page_runs;
};
hipError_t launch_feature_descriptors(const FeatureDescParams& p, int head_dim, hipStream_t s);

hipError_t launch_chrono_sum(const float* x, float* out, int64_t outer, int fines, int64_t inner,
                             hipStream_t s);

// Pending statistics of the regularized writer, in seal order: for block blk
// (fine slot first_slot + blk) pending = stats (first fine of a pending run)
// or pending + stats; a block that completes a page (reset_pages) has its
// stats entry overwritten by the page's sums, then the run restarts.
struct AssocPendingParams {
  float* gram; float* cross;            // [count * B][H][D][D] (in place)
  float* pending_gram; float* pending_cross;   // [B][H][D][D]
  int count, B, H, first_slot, group, reset_pages;
};
hipError_t launch_assoc_pending(const AssocPendingParams& p, int head_dim, hipStream_t s);
// The same in-order sums over dd elements per (b, h); cross / pending_cross
// may be null (one statistic).
hipError_t launch_pending_sums(const AssocPendingParams& p, int dd, hipStream_t s);

// h [B, T, H, D] (strides h_s), read_z element strides z_s (b, t, h, page),
// zero for broadcast axes; out bf16 [B, T, H, P, D] contiguous.
struct FeatureCoeffParams {
  const bf16_t* h; const bf16_t* z;
  int64_t h_s[3], z_s[4];
  int B, T, H, P;
  bf16_t* out;
};
hipError_t launch_feature_coeff(const FeatureCoeffParams& p, int head_dim, hipStream_t s);

// Channel-given selected contraction: channel [B, Q, H, M, D] bf16, ids
// [B, Q, H, M] int64, bank [BB, H, S, D, D] bf16 (C rows d, columns e; batch b
// reads bank b % BB), all contiguous.
struct SelectedParams {
  const bf16_t* channel; const int64_t* ids; const bf16_t* bank;
  int B, Q, H, M, BB, S;
  bf16_t* out;            // forward: [B, Q, H, D]
  const bf16_t* grad;     // backward: [B, Q, H, D]
  bf16_t* grad_channel;   // [B, Q, H, M, D] (nullable)
  bf16_t* grad_bank;      // [BB, H, S, D, D] (nullable)
};
hipError_t launch_selected_numerator(const SelectedParams& p, int head_dim, hipStream_t s);
hipError_t launch_selected_numerator_bwd(const SelectedParams& p, int head_dim, hipStream_t s);



}  // namespace tao
