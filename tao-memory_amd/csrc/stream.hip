// Native per-token decode driver (the host half of the decode step).
//
// Mirrors the reference's per-call control flow for a single new token
// (tao_attention_decode -> StreamCache.process -> LayerState._read_progressive
// -> _read_reused / HistoryRegionGraph.run -> seal; operator.py:130-138,
// tao_stream.py:196-249, 919-969, history_region_graph.py:66-113) in C++, so
// one ctypes call per token issues every launch: a route refresh on turn
// positions, the fused decode step (eagerly, or replayed within a graph
// epoch: a recorded argument block dispatched directly or a hipGraph), and
// the seal (writer + epilogue) when the local window reaches serve_limit; a
// seal that completes a page also builds its value matrix and refolds the
// coarse read when the state carries the coarse value branch.
// Every count is a closed form of the cursor (the same formulas as the
// Python host's schedule module).
#include <algorithm>
#include <cstring>
#include <vector>

#include "schedule.h"
#include "tao_launch.h"

extern "C" int tao_route(const tao_state_dev* st, const void* raw_q_row, const int64_t* rq_s,
                         int32_t completed, int32_t pending, int32_t coarse, int32_t selected,
                         void* stream);
extern "C" int tao_fold_route(const tao_state_dev* st, int32_t selected, void* stream);
extern "C" int tao_page_coarse(const tao_state_dev* st, int32_t first_page, int32_t count,
                               void* stream);
extern "C" int tao_fold_coarse(const tao_state_dev* st, int32_t completed, void* stream);
extern "C" int tao_write_fine(const tao_state_dev* st, const tao_tokens* tok, int64_t new_base,
                              const int64_t* start_pos, int32_t first_slot, int32_t count,
                              void* stream);
extern "C" int tao_seal_epilogue(const tao_state_dev* st, int32_t slot, int32_t pages,
                                 int32_t recompute, void* stream);
extern "C" int tao_graph_create(const tao_state_dev* st, const tao_fusion* fu, int32_t selected,
                                void* staging, void* out_stage, void* stream, void** graph_out);
extern "C" int tao_graph_launch(void* graph, const tao_tokens* tok, void* stream);
extern "C" int tao_graph_destroy(void* graph);

namespace {

using tao::sched::fines_at;
using tao::sched::first_turn;
using tao::sched::is_turn;
using tao::sched::local_len_at;
using tao::sched::serve_limit;

// Eager steps of an epoch before its capture (history_region_graph.py:90).
constexpr int kWarmSteps = 3;

enum Action { kUninitialized = 0, kEagerWarm, kCaptureReplay, kReplay, kRouteCopy, kInvalidate };

// One epoch of the decode graph (HistoryRegionGraph, history_region_graph.py:
// 10-113): the non-refresh steps of one state version, route size and
// fusion parameter set. The captured step is either a recorded kernel
// argument block dispatched directly (use_graph 1) or a hipGraph (2).
struct Epoch {
  bool open = false;
  int64_t version = -1;        // fines_at(cursor) when the epoch opened
  int32_t selected = -1;
  tao_fusion fusion{};
  int32_t warm = 0;
  bool recorded = false;       // use_graph 1: rec holds the captured step
  tao::DecodeParams rec{};
  void* graph = nullptr;       // use_graph 2
  int64_t stats[TAO_GRAPH_STATS] = {};
};

struct Stream {
  tao_state_dev st;
  tao_stream_cfg cfg;
  int64_t position = 0;
  int32_t route_coarse = 0, route_size = 0;
  void* staging = nullptr;
  void* out_stage = nullptr;
  Epoch ep;
  int64_t* seal_start = nullptr;   // device int64 (first word of the plan region)
  int64_t seal_host = 0;           // host copy staged by the seal's upload
};

int stream_fail(int code, const char* msg) {
  tao::set_error(msg);
  return code;
}

bool same_fusion(const tao_fusion& a, const tao_fusion& b) {
  return a.fusion_a == b.fusion_a && a.fusion_b == b.fusion_b && a.dtype == b.dtype &&
         a.gain == b.gain && a.coarse_on == b.coarse_on && a.fine_on == b.fine_on &&
         std::memcmp(a.a_s, b.a_s, sizeof(a.a_s)) == 0 &&
         std::memcmp(a.b_s, b.b_s, sizeof(a.b_s)) == 0;
}

void drop_graph(Stream* s) {
  Epoch& ep = s->ep;
  if (ep.graph) tao_graph_destroy(ep.graph);
  ep.graph = nullptr;
  ep.recorded = false;
}

// HistoryRegionGraph.invalidate (history_region_graph.py:39-57): counted
// once per open epoch. The caller's stream order keeps queued replays valid:
// nothing they read is freed here (the staging and output buffers belong to
// the caller; a destroyed hipGraphExec's queued launches complete).
void end_epoch(Stream* s, int reason) {
  Epoch& ep = s->ep;
  if (!ep.open) return;
  drop_graph(s);
  ep.open = false;
  ep.version = -1;
  ep.selected = -1;
  ep.warm = 0;
  ep.stats[TAO_GS_INVALIDATIONS] += 1;
  ep.stats[TAO_GS_REASON0 + reason] += 1;
  ep.stats[TAO_GS_LAST_ACTION] = kInvalidate;
  ep.stats[TAO_GS_LAST_REASON] = reason;
}

// HistoryRegionGraph.update_routes (history_region_graph.py:56-64), called
// by every route refresh (tao_stream.py:358-359).
void route_update(Stream* s, int32_t selected) {
  Epoch& ep = s->ep;
  if (!ep.open) return;
  if (selected != ep.selected) {
    end_epoch(s, TAO_GRAPH_SELECTED_SHAPE);
    return;
  }
  ep.stats[TAO_GS_ID_COPIES] += 1;
  ep.stats[TAO_GS_LAST_ACTION] = kRouteCopy;
}

// Route refresh due at the stream's cursor (before its decode step).
int pre_step(Stream* s, const tao_tokens* tok, void* stream, int* refreshed) {
  const tao_stream_cfg& c = s->cfg;
  const int64_t pos = s->position;
  const int64_t fines = fines_at(c, pos);
  *refreshed = 0;
  if (fines > 0 && is_turn(c, pos)) {
    const int64_t completed = fines / c.coarse_group, pending = fines % c.coarse_group;
    int64_t coarse64 = 0, eligible = 0, selected64 = 0;
    tao::sched::routed_counts(c, completed, pending, &coarse64, &eligible, &selected64);
    const int32_t coarse = (int32_t)coarse64, selected = (int32_t)selected64;
    const int64_t rq_s[2] = {tok->rq_s[0], tok->rq_s[2]};
    const int rc = tao::refresh_fold_at(&s->st, tok->raw_q, rq_s, (int32_t)completed,
                                        (int32_t)pending, coarse, selected, tao::TurnGate{},
                                        stream);
    if (rc) return rc;
    s->route_coarse = coarse;
    s->route_size = selected;
    *refreshed = 1;
    route_update(s, selected);
  }
  return TAO_OK;
}

// Seal due after the step at the stream's cursor; advances the cursor.
int post_step(Stream* s, const tao_tokens* tok, void* stream, int* sealed) {
  const tao_stream_cfg& c = s->cfg;
  const int64_t pos = s->position;
  const int64_t fines = fines_at(c, pos);
  const int64_t limit = c.local_keep + c.fine_tokens;
  *sealed = 0;
  if (local_len_at(c, pos) + 1 == limit) {
    s->seal_host = pos + 1 - limit;
    hipError_t e = hipMemcpyAsync(s->seal_start, &s->seal_host, sizeof(int64_t),
                                  hipMemcpyHostToDevice, (hipStream_t)stream);
    if (e != hipSuccess) return stream_fail((int)e, "seal start upload");
    int rc = tao_write_fine(&s->st, tok, pos + 1, s->seal_start, (int32_t)fines, 1, stream);
    if (!rc) rc = tao_seal_epilogue(&s->st, (int32_t)fines,
                                    (int32_t)(fines / c.coarse_group + 1), 1, stream);
    // New page weights and segment weights: refold the current route.
    if (!rc) rc = tao_fold_route(&s->st, s->route_size, stream);
    // A completed page: its value matrix, then the coarse read over all pages.
    // (The regularized writer's seal already wrote the page's matrix.)
    if (!rc && s->st.page_c && fines % c.coarse_group == c.coarse_group - 1) {
      const int32_t page = (int32_t)(fines / c.coarse_group);
      if (!s->st.pending_gram) rc = tao_page_coarse(&s->st, page, 1, stream);
      if (!rc) rc = tao_fold_coarse(&s->st, page + 1, stream);
    }
    if (rc) return rc;
    *sealed = 1;
    end_epoch(s, TAO_GRAPH_SEAL);     // append_fine (tao_stream.py:444-445)
  }
  s->position = pos + 1;
  return TAO_OK;
}

// One non-refresh step under use_graph (HistoryRegionGraph.run,
// history_region_graph.py:66-113). *staged = 1 when the heads are in
// out_stage (capture or replay), 0 when they are in out (eager warm step).
int region_step(Stream* s, const tao_tokens* tok, const tao_fusion* f, int32_t selected,
                void* out, const int64_t* out_s, void* stream, int* staged, int* captured) {
  Epoch& ep = s->ep;
  const int64_t version = fines_at(s->cfg, s->position);
  if (ep.open && (ep.version != version || ep.selected != selected || !same_fusion(ep.fusion, *f)))
    end_epoch(s, TAO_GRAPH_EPOCH_CHANGE);
  if (!ep.open) {
    // A new epoch stages the current route ids (history_region_graph.py:78-89).
    ep.open = true;
    ep.version = version;
    ep.selected = selected;
    ep.fusion = *f;
    ep.warm = 0;
    ep.stats[TAO_GS_EPOCHS] += 1;
    ep.stats[TAO_GS_ID_COPIES] += 1;
  }
  *staged = 0;
  *captured = 0;
  if (ep.warm < kWarmSteps) {
    const int rc = tao::decode_step_at(&s->st, tok, f, selected, out, out_s, stream, s->position);
    if (rc) return rc;
    ep.warm += 1;
    ep.stats[TAO_GS_EAGER_WARM] += 1;
    ep.stats[TAO_GS_LAST_ACTION] = kEagerWarm;
    return TAO_OK;
  }
  const tao_stream_cfg& c = s->cfg;
  const int64_t stage_s[3] = {(int64_t)s->st.heads * s->st.head_dim, 0, (int64_t)s->st.head_dim};
  int rc = TAO_OK;
  if (c.use_graph == 2) {
    if (!ep.graph) {
      rc = tao_graph_create(&s->st, f, selected, s->staging, s->out_stage, stream, &ep.graph);
      if (rc) return rc;
      *captured = 1;
    }
    rc = tao_graph_launch(ep.graph, tok, stream);
  } else {
    if (!ep.recorded) {
      rc = tao::decode_record(&s->st, tok, f, selected, s->out_stage, stage_s, &ep.rec);
      if (rc) return rc;
      ep.recorded = true;
      *captured = 1;
    }
    rc = tao::decode_replay(ep.rec, tok, s->st.head_dim, selected, s->position, stream);
  }
  if (rc) return rc;
  if (*captured) ep.stats[TAO_GS_CAPTURES] += 1;
  ep.stats[TAO_GS_REPLAYS] += 1;
  ep.stats[TAO_GS_LAST_ACTION] = *captured ? kCaptureReplay : kReplay;
  *staged = 1;
  return TAO_OK;
}

// The reference's prefill path over an open epoch (tao_stream.py:196-249):
// the refreshes of positions [s->position, to) copy route ids (or end the
// epoch on a new route size) until the first seal, which ends it.
void epoch_advance(Stream* s, int64_t to) {
  const tao_stream_cfg& c = s->cfg;
  for (int64_t t = s->position; t < to && s->ep.open; ++t) {
    const int64_t fines = fines_at(c, t);
    if (fines != s->ep.version) {
      end_epoch(s, TAO_GRAPH_SEAL);
      break;
    }
    if (fines > 0 && is_turn(c, t)) {
      int64_t coarse = 0, eligible = 0, selected = 0;
      tao::sched::routed_counts(c, fines / c.coarse_group, fines % c.coarse_group, &coarse,
                                &eligible, &selected);
      route_update(s, (int32_t)selected);
    }
  }
  if (s->ep.open && fines_at(c, to) != s->ep.version) end_epoch(s, TAO_GRAPH_SEAL);
}

struct Batch {
  std::vector<Stream*> reqs;
  std::vector<tao::BatchReq> host_table;   // staging of the device table upload
  tao::BatchReq* table = nullptr;          // caller's device memory
  int heads = 0, head_dim = 0, keep = 0, fine = 0, group = 0, coarse_values = 0;
};

// The device table entry of one request: its buffers as its driver holds them.
tao::BatchReq table_entry(const tao_state_dev& st) {
  const tao::WorkspaceLayout lay =
      tao::workspace_layout(st.batch, st.heads, st.head_dim, st.sel_cap, 0);
  tao::BatchReq t{};
  t.ring_k = (bf16_t*)st.ring_k;
  t.ring_v = (bf16_t*)st.ring_v;
  t.ring_raw = (bf16_t*)st.ring_raw;
  t.fold_g = (const float*)st.fold_g;
  t.fold_den = (const float*)st.fold_den;
  t.coarse_g = (const float*)st.coarse_g;
  t.header = st.header;
  t.parts = (float*)((char*)st.workspace + lay.parts_off);
  return t;
}

bool same_entry(const tao::BatchReq& a, const tao::BatchReq& b) {
  return a.ring_k == b.ring_k && a.ring_v == b.ring_v && a.ring_raw == b.ring_raw &&
         a.fold_g == b.fold_g && a.fold_den == b.fold_den && a.coarse_g == b.coarse_g &&
         a.header == b.header && a.parts == b.parts;
}

int fill_table(Batch* b, void* stream) {
  for (size_t r = 0; r < b->reqs.size(); ++r) b->host_table[r] = table_entry(b->reqs[r]->st);
  const hipError_t e = hipMemcpyAsync(b->table, b->host_table.data(),
                                      b->host_table.size() * sizeof(tao::BatchReq),
                                      hipMemcpyHostToDevice, (hipStream_t)stream);
  return e == hipSuccess ? TAO_OK : stream_fail((int)e, "batch table upload");
}

// Batch row r of the call's operands as a one-request token view.
tao_tokens row_tokens(const tao_tokens* tok, int r) {
  tao_tokens t = *tok;
  t.q = (const bf16_t*)tok->q + r * tok->q_s[0];
  t.k = (const bf16_t*)tok->k + r * tok->k_s[0];
  t.v = (const bf16_t*)tok->v + r * tok->v_s[0];
  t.raw_q = (const bf16_t*)tok->raw_q + r * tok->rq_s[0];
  t.raw_k = (const bf16_t*)tok->raw_k + r * tok->rk_s[0];
  t.tokens = 1;
  return t;
}

}  // namespace

extern "C" {

int tao_stream_open(const tao_state_dev* st, const tao_stream_cfg* cfg, int64_t position,
                    int32_t route_coarse, int32_t route_size, void* staging, void* out_stage,
                    void** handle) {
  if (!st || !cfg || !handle) return stream_fail(TAO_E_ARGUMENT, "null stream argument");
  if (cfg->route_period <= 0 || cfg->fine_tokens <= 0 || cfg->coarse_group <= 0)
    return stream_fail(TAO_E_ARGUMENT, "invalid stream geometry");
  Stream* s = new Stream();
  s->st = *st;
  s->cfg = *cfg;
  s->position = position;
  s->route_coarse = route_coarse;
  s->route_size = route_size;
  s->staging = staging;
  s->out_stage = out_stage;
  s->ep.stats[TAO_GS_LAST_REASON] = -1;
  const tao::WorkspaceLayout lay =
      tao::workspace_layout(st->batch, st->heads, st->head_dim, st->sel_cap, 0);
  s->seal_start = (int64_t*)((char*)st->workspace + lay.plan_off);
  *handle = s;
  return TAO_OK;
}

int tao_stream_sync(void* handle, const tao_state_dev* st, int64_t position,
                    int32_t route_coarse, int32_t route_size) {
  if (!handle) return stream_fail(TAO_E_ARGUMENT, "null stream");
  Stream* s = (Stream*)handle;
  if (position < s->position) end_epoch(s, TAO_GRAPH_EPOCH_CHANGE);
  else epoch_advance(s, position);
  if (st && std::memcmp(st, &s->st, sizeof(*st)) != 0) {
    end_epoch(s, TAO_GRAPH_EPOCH_CHANGE);
    drop_graph(s);
    s->st = *st;
    const tao::WorkspaceLayout lay =
        tao::workspace_layout(st->batch, st->heads, st->head_dim, st->sel_cap, 0);
    s->seal_start = (int64_t*)((char*)st->workspace + lay.plan_off);
  }
  s->position = position;
  s->route_coarse = route_coarse;
  s->route_size = route_size;
  return TAO_OK;
}

namespace {

bool seal_after(const tao_stream_cfg& c, int64_t pos) {
  return local_len_at(c, pos) + 1 == c.local_keep + c.fine_tokens;
}

// A route refresh at a turn in pos's state version keeps the current route's
// coarse count and size (routed_counts of the version equal them), so a
// device-cursor step may carry it gated on the device cursor: the route
// kernels' counts and the step's route size hold for every turn of the
// version.
bool route_kept(const Stream* s, int64_t pos) {
  const tao_stream_cfg& c = s->cfg;
  const int64_t fines = fines_at(c, pos);
  if (fines <= 0) return false;
  int64_t coarse = 0, eligible = 0, selected = 0;
  tao::sched::routed_counts(c, fines / c.coarse_group, fines % c.coarse_group, &coarse,
                            &eligible, &selected);
  return coarse == s->route_coarse && selected == s->route_size;
}

// The token at `pos` can run as a device-cursor step: no seal after it, and
// either no route refresh before it or one that keeps the route.
bool replayable_at(const Stream* s, int64_t pos) {
  const tao_stream_cfg& c = s->cfg;
  if (seal_after(c, pos)) return false;
  const bool refresh = fines_at(c, pos) > 0 && is_turn(c, pos);
  return !refresh || route_kept(s, pos);
}

// The fusion flags of a step at `pos` (as tao_stream_decode sets them).
tao_fusion step_fusion(const Stream* s, const tao_fusion& fu, int64_t pos) {
  const int64_t fines = fines_at(s->cfg, pos);
  tao_fusion f = fu;
  f.coarse_on = s->st.page_c != nullptr && fines >= s->cfg.coarse_group;
  f.fine_on = fines > 0;
  return f;
}

}  // namespace

int tao_stream_plan_step(void* handle, int64_t* info) {
  if (!handle || !info) return stream_fail(TAO_E_ARGUMENT, "null plan argument");
  const Stream* s = (const Stream*)handle;
  const tao_stream_cfg& c = s->cfg;
  const int64_t pos = s->position, fines = fines_at(c, pos);
  info[0] = pos;
  info[1] = fines > 0 && is_turn(c, pos);
  info[2] = seal_after(c, pos);
  info[3] = fines > 0 ? s->route_size : 0;
  info[4] = fines > 0;
  info[5] = s->st.page_c != nullptr && fines >= c.coarse_group;
  info[6] = route_kept(s, pos);
  return TAO_OK;
}

int tao_stream_graph_step(void* handle, const tao_tokens* tok, const tao_fusion* fu, void* out,
                          const int64_t* out_s, void* stream) {
  if (!handle || !tok || !fu) return stream_fail(TAO_E_ARGUMENT, "null decode argument");
  Stream* s = (Stream*)handle;
  const tao_stream_cfg& c = s->cfg;
  const int64_t pos = s->position;
  if (!replayable_at(s, pos))
    return stream_fail(TAO_E_ARGUMENT,
                       "the next token seals or changes its route: it cannot be a device-cursor step");
  const int64_t fines = fines_at(c, pos);
  if (route_kept(s, pos)) {
    // The version's refresh, run on the device only when the cursor the step
    // reads is a turn of this layer (pre_step's route + fold).
    const tao::TurnGate gate{s->st.header, (long long)first_turn(c), (long long)c.route_period,
                             (long long)serve_limit(c)};
    const int64_t rq_s[2] = {tok->rq_s[0], tok->rq_s[2]};
    const int rc = tao::refresh_fold_at(&s->st, tok->raw_q, rq_s,
                                        (int32_t)(fines / c.coarse_group),
                                        (int32_t)(fines % c.coarse_group), s->route_coarse,
                                        s->route_size, gate, stream);
    if (rc) return rc;
  }
  const tao_fusion f = step_fusion(s, *fu, pos);
  const int32_t selected = fines > 0 ? s->route_size : 0;
  return tao::decode_step_at(&s->st, tok, &f, selected, out, out_s, stream, -1);
}

int tao_stream_advance(void* handle, int64_t count) {
  if (!handle) return stream_fail(TAO_E_ARGUMENT, "null stream");
  Stream* s = (Stream*)handle;
  if (count < 0) return stream_fail(TAO_E_ARGUMENT, "negative step count");
  for (int64_t i = 0; i < count; ++i)
    if (!replayable_at(s, s->position + i))
      return stream_fail(TAO_E_ARGUMENT, "advance over a seal or a route change");
  // A device-cursor step keeps the route size and counts, which is all the
  // driver tracks of a refresh (epoch_advance books its route update).
  epoch_advance(s, s->position + count);
  s->position += count;
  return TAO_OK;
}

int tao_stream_decode(void* handle, const tao_tokens* tok, const tao_fusion* fu, void* out,
                      const int64_t* out_s, void* stream, int64_t* info) {
  if (!handle || !tok || !fu || !info) return stream_fail(TAO_E_ARGUMENT, "null decode argument");
  Stream* s = (Stream*)handle;
  const tao_stream_cfg& c = s->cfg;
  const int64_t pos = s->position;
  const int64_t fines = fines_at(c, pos);
  int refreshed = 0, sealed = 0;
  int rc = pre_step(s, tok, stream, &refreshed);
  if (rc) return rc;
  const int32_t selected = fines > 0 ? s->route_size : 0;
  const bool coarse_values = s->st.page_c != nullptr;
  tao_fusion f = *fu;
  f.coarse_on = coarse_values && fines >= c.coarse_group;   // a completed page exists
  f.fine_on = fines > 0;
  int staged = 0, captured = 0;
  // The graph serves the memo-backed index-only read of non-refresh steps
  // (tao_stream.py:238-249); refresh steps run eagerly.
  if (c.use_graph && !coarse_values && fines > 0 && !refreshed) {
    if (!s->out_stage)
      return stream_fail(TAO_E_ARGUMENT, "decode graph needs the output buffer");
    rc = region_step(s, tok, &f, selected, out, out_s, stream, &staged, &captured);
  } else {
    rc = tao::decode_step_at(&s->st, tok, &f, selected, out, out_s, stream, pos);
  }
  if (rc) return rc;
  rc = post_step(s, tok, stream, &sealed);
  if (rc) return rc;
  info[0] = s->position;
  info[1] = s->route_coarse;
  info[2] = s->route_size;
  info[3] = refreshed;
  info[4] = sealed;
  info[5] = staged;
  info[6] = captured;
  return TAO_OK;
}

size_t tao_batch_table_bytes(int32_t count) {
  return count > 0 ? (size_t)count * sizeof(tao::BatchReq) : 0;
}

int tao_batch_open(void* const* handles, int32_t count, void* table, size_t table_bytes,
                   void* stream, void** batch) {
  if (!handles || count <= 0 || !table || !batch)
    return stream_fail(TAO_E_ARGUMENT, "null batch argument");
  if (table_bytes < tao_batch_table_bytes(count))
    return stream_fail(TAO_E_WORKSPACE, "batch table smaller than tao_batch_table_bytes()");
  Batch* b = new Batch();
  for (int32_t r = 0; r < count; ++r) {
    Stream* s = (Stream*)handles[r];
    if (!s) {
      delete b;
      return stream_fail(TAO_E_ARGUMENT, "null stream in the batch");
    }
    const tao_state_dev& st = s->st;
    const char* why = nullptr;
    if (st.batch != 1) why = "batched decode takes states of batch 1";
    else if (!b->reqs.empty()) {
      const tao_state_dev& f = b->reqs[0]->st;
      const tao_stream_cfg& c0 = b->reqs[0]->cfg;
      if (st.heads != f.heads || st.head_dim != f.head_dim || st.local_keep != f.local_keep ||
          st.fine_tokens != f.fine_tokens || st.coarse_group != f.coarse_group ||
          (st.page_c == nullptr) != (f.page_c == nullptr) ||
          s->cfg.local_keep != c0.local_keep || s->cfg.fine_tokens != c0.fine_tokens)
        why = "batched states must share heads, head width, geometry and coarse branch";
      for (Stream* o : b->reqs)
        if (o == s) why = "a state appears twice in the batch";
    }
    if (why) {
      delete b;
      return stream_fail(TAO_E_ARGUMENT, why);
    }
    b->reqs.push_back(s);
  }
  const tao_state_dev& f = b->reqs[0]->st;
  b->heads = f.heads;
  b->head_dim = f.head_dim;
  b->keep = f.local_keep;
  b->fine = f.fine_tokens;
  b->group = f.coarse_group;
  b->coarse_values = f.page_c != nullptr;
  b->table = (tao::BatchReq*)table;
  b->host_table.resize(count);
  const int rc = fill_table(b, stream);
  if (rc) {
    delete b;
    return rc;
  }
  *batch = b;
  return TAO_OK;
}

int tao_batch_sync(void* batch, void* stream) {
  if (!batch) return stream_fail(TAO_E_ARGUMENT, "null batch");
  Batch* b = (Batch*)batch;
  // Host staging may still be read by the previous upload: wait for it.
  if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess)
    return stream_fail(TAO_E_ARGUMENT, "batch sync: stream error");
  return fill_table(b, stream);
}

int tao_batch_decode(void* batch, const tao_tokens* tok, const tao_fusion* fu, void* out,
                     const int64_t* out_s, void* stream, int64_t* info) {
  if (!batch || !tok || !fu || !out || !out_s || !info)
    return stream_fail(TAO_E_ARGUMENT, "null batch decode argument");
  Batch* b = (Batch*)batch;
  const int R = (int)b->reqs.size();
  if (tok->tokens != 1) return stream_fail(TAO_E_SHAPE, "batched decode takes one token per request");
  if (!tok->q || !tok->k || !tok->v || !tok->raw_q || !tok->raw_k)
    return stream_fail(TAO_E_ARGUMENT, "null token operand");
  if (!fu->fusion_a || !fu->fusion_b ||
      (fu->dtype != TAO_BF16 && fu->dtype != TAO_FP32 && fu->dtype != TAO_FP16))
    return stream_fail(TAO_E_ARGUMENT, "invalid fusion parameters");
  // A member whose buffers moved since the table was uploaded (its host
  // re-synced the driver but not the batch) gets the table refreshed first:
  // the step kernels must never follow a stale buffer address.
  for (int r = 0; r < R; ++r) {
    if (!same_entry(b->host_table[r], table_entry(b->reqs[r]->st))) {
      const int rc = tao_batch_sync(b, stream);
      if (rc) return rc;
      break;
    }
  }
  for (int r = 0; r < R; ++r) {
    Stream* s = b->reqs[r];
    const tao_tokens t = row_tokens(tok, r);
    int refreshed = 0;
    const int rc = pre_step(s, &t, stream, &refreshed);
    if (rc) return rc;
    info[4 * r] = refreshed;
  }
  tao::BatchStepParams p{};
  auto view = [](const void* ptr, const int64_t* st) {
    tao::TokView v;
    v.p = (const bf16_t*)ptr;
    v.sb = st[0];
    v.st = st[1];
    v.sh = st[2];
    return v;
  };
  p.q = view(tok->q, tok->q_s);
  p.k = view(tok->k, tok->k_s);
  p.v = view(tok->v, tok->v_s);
  p.rq = view(tok->raw_q, tok->rq_s);
  p.rk = view(tok->raw_k, tok->rk_s);
  p.fa = fu->fusion_a;
  p.fb = fu->fusion_b;
  p.f_dtype = fu->dtype;
  for (int i = 0; i < 3; ++i) { p.fa_s[i] = fu->a_s[i]; p.fb_s[i] = fu->b_s[i]; }
  p.gain = fu->gain;
  p.out = (bf16_t*)out;
  p.out_sb = out_s[0];
  p.out_sh = out_s[2];
  p.table = b->table;
  p.R = R;
  p.H = b->heads;
  p.keep = b->keep;
  p.fine = b->fine;
  p.group = b->group;
  p.coarse_values = b->coarse_values;
  const hipError_t e = tao::launch_batch_step(p, b->head_dim, (hipStream_t)stream);
  if (e != hipSuccess) return stream_fail((int)e, "batched decode step launch");
  for (int r = 0; r < R; ++r) {
    Stream* s = b->reqs[r];
    const tao_tokens t = row_tokens(tok, r);
    int sealed = 0;
    const int rc = post_step(s, &t, stream, &sealed);
    if (rc) return rc;
    info[4 * r + 1] = sealed;
    info[4 * r + 2] = s->route_coarse;
    info[4 * r + 3] = s->route_size;
  }
  return TAO_OK;
}

int tao_batch_close(void* batch) {
  delete (Batch*)batch;
  return TAO_OK;
}

int tao_stream_invalidate(void* handle, int32_t reason) {
  if (!handle) return TAO_OK;
  if (reason < 0 || reason >= TAO_GRAPH_REASONS)
    return stream_fail(TAO_E_ARGUMENT, "unknown graph invalidation reason");
  Stream* s = (Stream*)handle;
  end_epoch(s, reason);
  drop_graph(s);
  return TAO_OK;
}

int tao_stream_graph_stats(void* handle, int64_t* stats, int32_t n) {
  if (!handle || !stats || n < 0) return stream_fail(TAO_E_ARGUMENT, "null graph stats argument");
  const Stream* s = (const Stream*)handle;
  int64_t all[TAO_GRAPH_STATS];
  std::memcpy(all, s->ep.stats, sizeof(all));
  all[TAO_GS_ACTIVE_GRAPH] = (s->ep.graph != nullptr || s->ep.recorded) ? 1 : 0;
  all[TAO_GS_ACTIVE_EPOCH] = s->ep.open ? 1 : 0;
  all[TAO_GS_EPOCH_VERSION] = s->ep.open ? s->ep.version : -1;
  all[TAO_GS_WARM] = s->ep.warm;
  std::memcpy(stats, all, sizeof(int64_t) * (size_t)std::min<int32_t>(n, TAO_GRAPH_STATS));
  return TAO_OK;
}

int tao_stream_release(void* handle) { return tao_stream_invalidate(handle, TAO_GRAPH_REQUEST_END); }

int tao_stream_close(void* handle) {
  if (!handle) return TAO_OK;
  Stream* s = (Stream*)handle;
  drop_graph(s);
  delete s;
  return TAO_OK;
}

}  // extern "C"
