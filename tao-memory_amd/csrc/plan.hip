// Native builder of the tao_prefill plan (host code).
//
// Replaces the host side of the reference's prefill loop
// (tao_attention_prefill, operator.py:100-127, with StreamCache.process,
// tao_stream.py:919-979, per chunk, and _read_progressive's turn split,
// tao_stream.py:196-227): it lays out every chunk's local-attention tiles,
// the seal blocks, every route turn and every read tile of a prompt as the
// int64 plan that tao_prefill validates and executes (enum tao_plan_field).
#include <vector>

#include "schedule.h"
#include "tao_launch.h"

namespace {

constexpr int64_t kReadTile = 32;    // queries per read tile (one wave)

}  // namespace

extern "C" int tao_prefill_plan(const tao_stream_cfg* cfg, int64_t pos0, int64_t tokens,
                                int32_t route_coarse, int32_t route_size, int32_t outputs,
                                int64_t* plan, int64_t plan_cap, int64_t* info) {
  using namespace tao::sched;
  if (!cfg || !info) {
    tao::set_error("null plan argument");
    return TAO_E_ARGUMENT;
  }
  const tao_stream_cfg& c = *cfg;
  if (c.fine_tokens <= 0 || c.local_keep < 0 || c.coarse_group <= 0 || c.route_period <= 0 ||
      pos0 < 0 || tokens < 0) {
    tao::set_error("invalid plan geometry");
    return TAO_E_ARGUMENT;
  }
  const int64_t group = c.coarse_group;
  const int64_t end = pos0 + tokens;
  const int64_t f0 = fines_at(c, pos0), f1 = fines_at(c, end);
  struct Chunk { int64_t start, width, epoch; };
  std::vector<Chunk> chunks;
  for (int64_t start = pos0; start < end;) {
    const int64_t w = next_chunk(c, start, end - start);
    chunks.push_back({start, w, fines_at(c, start)});
    start += w;
  }
  std::vector<int64_t> attn, reads, turns;
  int64_t history_chunks = 0;
  for (const Chunk& ch : chunks) history_chunks += ch.epoch > 0;
  if (outputs)
    attention_tiles(c, pos0, tokens, [&](int64_t row, int64_t n, int64_t key_start) {
      attn.insert(attn.end(), {row, n, key_start});
    });
  // Epochs read by this call plus the published final epoch.
  int64_t first_epoch = 0;
  if (f1 >= 1) {
    first_epoch = f1;
    for (const Chunk& ch : chunks)
      if (ch.epoch >= 1 && ch.epoch < first_epoch) first_epoch = ch.epoch;
    if (first_epoch < 1) first_epoch = 1;
    if (!outputs) first_epoch = f1;
  }
  int64_t slot = 0, slot_m = route_size;
  int64_t r_coarse = route_coarse, r_size = route_size;
  bool have_last = false;
  int64_t last[6] = {0, 0, 0, 0, 0, 0};
  for (const Chunk& ch : chunks) {
    for (int64_t off = 0; off < ch.width;) {
      const int64_t sub = ch.start + off;
      int64_t count = next_turn(c, sub) - sub;
      if (count > ch.width - off) count = ch.width - off;
      const bool refresh = is_turn(c, sub);
      off += count;
      if (ch.epoch == 0) {
        if (outputs)
          for (int64_t qs = sub; qs < sub + count; qs += kReadTile) {
            const int64_t n = sub + count - qs;
            reads.insert(reads.end(), {qs - pos0, n < kReadTile ? n : kReadTile, 0, 0, 0, 0, 0, 0});
          }
        continue;
      }
      if (refresh) {
        const int64_t completed = ch.epoch / group, pending = ch.epoch % group;
        int64_t coarse, eligible, selected;
        routed_counts(c, completed, pending, &coarse, &eligible, &selected);
        have_last = true;
        const int64_t l[6] = {sub, ch.epoch, completed, pending, coarse, selected};
        for (int i = 0; i < 6; ++i) last[i] = l[i];
        if (outputs) {
          const int64_t index = (int64_t)turns.size() / 8 + 1;
          turns.insert(turns.end(), {sub - pos0, ch.epoch - first_epoch, completed, pending,
                                     coarse, selected, index, 0});
          slot = index;
          slot_m = selected;
        }
        r_coarse = coarse;
        r_size = selected;
      }
      if (outputs)
        for (int64_t qs = sub; qs < sub + count; qs += kReadTile) {
          const int64_t n = sub + count - qs;
          reads.insert(reads.end(), {qs - pos0, n < kReadTile ? n : kReadTile, slot, slot_m,
                                     ch.epoch - first_epoch, (ch.epoch / group) * group, 1,
                                     ch.epoch / group});
        }
    }
  }
  if (!outputs && have_last) {
    if (last[1] < first_epoch) first_epoch = last[1];
    turns.assign({last[0] - pos0, last[1] - first_epoch, last[2], last[3], last[4], last[5], 1, 1});
  } else if (!turns.empty()) {
    turns.back() = 1;
  }
  const int64_t n_epochs = f1 >= 1 ? f1 - first_epoch + 1 : 0;
  // Completed-page counts read by history chunks (coarse value branch).
  int64_t c_lo = 0, c_hi = 0;
  if (outputs)
    for (const Chunk& ch : chunks) {
      const int64_t completed = ch.epoch / group;
      if (completed < 1) continue;
      if (c_lo == 0 || completed < c_lo) c_lo = completed;
      if (completed > c_hi) c_hi = completed;
    }
  const int64_t limit = serve_limit(c);
  const int64_t keep = tokens < limit ? tokens : limit;
  const int64_t n_writes = f1 - f0;
  const int64_t len = TAO_PLAN_HEADER + (int64_t)attn.size() + n_writes + (int64_t)turns.size() +
                      (int64_t)reads.size();
  info[0] = len;
  info[1] = n_epochs;
  info[2] = (int64_t)turns.size() / 8;
  info[3] = r_coarse;
  info[4] = r_size;
  info[5] = f1 / group + 1;             // page capacity of the epoch pools
  info[6] = history_chunks;             // chunks that read history (fusion calls)
  info[7] = (int64_t)chunks.size();
  info[8] = c_lo;                       // coarse pool: first completed-page count
  info[9] = c_lo ? c_hi - c_lo + 1 : 0; // coarse pool: number of counts
  if (!plan) return TAO_OK;             // size query
  if (plan_cap < len) {
    tao::set_error("plan buffer too small");
    return TAO_E_WORKSPACE;
  }
  int64_t* h = plan;
  for (int i = 0; i < TAO_PLAN_HEADER; ++i) h[i] = 0;
  h[TAO_PLAN_POS0] = pos0;
  h[TAO_PLAN_ATTN_TILES] = (int64_t)attn.size() / 3;
  h[TAO_PLAN_WRITES] = n_writes;
  h[TAO_PLAN_FIRST_SLOT] = f0;
  h[TAO_PLAN_FIRST_PAGE] = f0 / group;
  h[TAO_PLAN_PAGES] = f1 / group - f0 / group;
  h[TAO_PLAN_FIRST_EPOCH] = first_epoch;
  h[TAO_PLAN_EPOCHS] = n_epochs;
  h[TAO_PLAN_TURNS] = (int64_t)turns.size() / 8;
  h[TAO_PLAN_READ_TILES] = (int64_t)reads.size() / 8;
  h[TAO_PLAN_RING_FIRST] = tokens - keep;
  h[TAO_PLAN_RING_COUNT] = keep;
  h[TAO_PLAN_RING_POS] = end - keep;
  int64_t* o = plan + TAO_PLAN_HEADER;
  for (int64_t v : attn) *o++ = v;
  for (int64_t f = f0; f < f1; ++f) *o++ = c.fine_tokens * f;
  for (int64_t v : turns) *o++ = v;
  for (int64_t v : reads) *o++ = v;
  return TAO_OK;
}

// Full-sequence read (tao_attention forward, operator.py:40-52): the tiling
// of read_training (tao_stream.py:668-757) and _local_training_corrected_4k
// (:760-787) as a tao_prefill plan for a fresh state. Tile t = tokens
// [F t, min(T, F t + F)) attends suffix-causally to keys from
// max(0, F t - local_keep) (the corrected-4k windows and the ragged fallback
// are the same windows), reads the first max(0, t - local_keep / F) sealed
// fines, and every query routes itself (route_interval = 1). The blocks the
// last tile can read are written; the ring is left empty.
extern "C" int tao_train_plan(const tao_stream_cfg* cfg, int64_t tokens, int64_t* plan,
                              int64_t plan_cap, int64_t* info) {
  using namespace tao::sched;
  if (!cfg || !info) {
    tao::set_error("null plan argument");
    return TAO_E_ARGUMENT;
  }
  const tao_stream_cfg& c = *cfg;
  if (c.fine_tokens <= 0 || c.local_keep < 0 || c.local_keep % c.fine_tokens ||
      c.coarse_group <= 0 || tokens < 0) {
    tao::set_error("invalid plan geometry");
    return TAO_E_ARGUMENT;
  }
  const int64_t ft = c.fine_tokens, group = c.coarse_group;
  const int64_t lag = c.local_keep / ft;                 // config.visibility_tiles
  const int64_t n_tiles = (tokens + ft - 1) / ft;
  const int64_t visible_max = n_tiles - 1 - lag > 0 ? n_tiles - 1 - lag : 0;
  std::vector<int64_t> attn, reads;
  int64_t history = 0, c_lo = 0, c_hi = 0;
  for (int64_t t = 0; t < n_tiles; ++t) {
    const int64_t s = t * ft, e = s + ft < tokens ? s + ft : tokens;
    const int64_t key_start = s > c.local_keep ? s - c.local_keep : 0;
    constexpr int64_t kTile = tao::sched::kAttnTile;
    for (int64_t qs = s; qs < e; qs += kTile)
      attn.insert(attn.end(), {qs, e - qs < kTile ? e - qs : kTile, key_start});
    const int64_t visible = t > lag ? t - lag : 0;
    int64_t coarse = 0, eligible = 0, selected = 0;
    if (visible) {
      routed_counts(c, visible / group, visible % group, &coarse, &eligible, &selected);
      ++history;
      const int64_t completed = visible / group;
      if (completed >= 1) {
        if (c_lo == 0 || completed < c_lo) c_lo = completed;
        if (completed > c_hi) c_hi = completed;
      }
    }
    for (int64_t qs = s; qs < e; qs += kReadTile) {
      const int64_t n = e - qs < kReadTile ? e - qs : kReadTile;
      if (visible)
        reads.insert(reads.end(), {qs, n, coarse, selected, visible - 1, (visible / group) * group,
                                   1, visible / group});
      else
        reads.insert(reads.end(), {qs, n, 0, 0, 0, 0, 0, 0});
    }
  }
  const int64_t len = TAO_PLAN_HEADER + (int64_t)attn.size() + visible_max + (int64_t)reads.size();
  info[0] = len;
  info[1] = visible_max;                    // epochs 1 .. visible_max
  info[2] = 0;                              // no turns
  info[3] = 0;
  info[4] = 0;
  info[5] = visible_max / group + 1;        // page capacity of the epoch pools
  info[6] = history;                        // tiles that read history
  info[7] = n_tiles;
  info[8] = c_lo;
  info[9] = c_lo ? c_hi - c_lo + 1 : 0;
  info[10] = visible_max;                   // fines written
  info[11] = (visible_max + 31) / 32;       // bitmask words per query
  if (!plan) return TAO_OK;
  if (plan_cap < len) {
    tao::set_error("plan buffer too small");
    return TAO_E_WORKSPACE;
  }
  int64_t* h = plan;
  for (int i = 0; i < TAO_PLAN_HEADER; ++i) h[i] = 0;
  h[TAO_PLAN_POS0] = 0;
  h[TAO_PLAN_ATTN_TILES] = (int64_t)attn.size() / 3;
  h[TAO_PLAN_WRITES] = visible_max;
  h[TAO_PLAN_FIRST_SLOT] = 0;
  h[TAO_PLAN_FIRST_PAGE] = 0;
  h[TAO_PLAN_PAGES] = visible_max / group;
  h[TAO_PLAN_FIRST_EPOCH] = visible_max ? 1 : 0;
  h[TAO_PLAN_EPOCHS] = visible_max;
  h[TAO_PLAN_TURNS] = 0;
  h[TAO_PLAN_READ_TILES] = (int64_t)reads.size() / 8;
  h[TAO_PLAN_RING_FIRST] = tokens;
  h[TAO_PLAN_RING_COUNT] = 0;
  h[TAO_PLAN_RING_POS] = tokens;
  h[TAO_PLAN_QUERY_ROUTES] = 1;
  int64_t* o = plan + TAO_PLAN_HEADER;
  for (int64_t v : attn) *o++ = v;
  for (int64_t f = 0; f < visible_max; ++f) *o++ = ft * f;
  for (int64_t v : reads) *o++ = v;
  return TAO_OK;
}
