// Closed forms of the streaming schedule (host code). Every count of the
// reference's lifecycle is a function of the causal cursor: the local window
// grows to serve_limit = local_keep + fine_tokens and then seals its oldest
// fine_tokens block (tao_stream.py:914-917, 959-967); route refreshes follow
// tao_stream.py:202-210 and the selected counts tao_stream.py:29-37.
#pragma once

#include <stdint.h>

#include "../../include/tao_memory.h"

// The route-size closed forms also run on the device (the fp32 full-sequence
// read derives each tile's counts in its kernel).
#if defined(__HIPCC__)
#define TAO_SCHED __host__ __device__ inline
#else
#define TAO_SCHED inline
#endif

namespace tao {
namespace sched {

inline int64_t serve_limit(const tao_stream_cfg& c) { return (int64_t)c.local_keep + c.fine_tokens; }

// Exact-local tokens held before the token at position p is appended.
inline int64_t local_len_at(const tao_stream_cfg& c, int64_t p) {
  const int64_t limit = serve_limit(c);
  return p < limit ? p : c.local_keep + (p - limit) % c.fine_tokens;
}

// Sealed fine memories after p tokens.
inline int64_t fines_at(const tao_stream_cfg& c, int64_t p) {
  const int64_t limit = serve_limit(c);
  return p < limit ? 0 : (p - limit) / c.fine_tokens + 1;
}

inline int64_t first_turn(const tao_stream_cfg& c) {
  return serve_limit(c) + (int64_t)c.layer_stagger * c.layer;
}

// Route refresh at position p (tao_stream.py:202-208).
inline bool is_turn(const tao_stream_cfg& c, int64_t p) {
  const int64_t ft = first_turn(c);
  return p == serve_limit(c) || (p >= ft && (p - ft) % c.route_period == 0);
}

// First refresh strictly after p (tao_stream.py:209-210).
inline int64_t next_turn(const tao_stream_cfg& c, int64_t p) {
  const int64_t ft = first_turn(c);
  if (p < ft) return ft;
  return ft + (int64_t)c.route_period * ((p - ft) / c.route_period + 1);
}

// budget(n) = min(n, ceil(sqrt(scale * n)) + offset) (config.py:54-60).
TAO_SCHED int64_t budget(const tao_stream_cfg& c, int64_t n) {
  if (n <= 0) return 0;
  const int64_t target = (int64_t)c.budget_root_scale * n;
  int64_t r = 0;
  while ((r + 1) * (r + 1) <= target) ++r;
  if (r * r < target) ++r;
  const int64_t b = r + c.budget_offset;
  return b < n ? b : n;
}

// (coarse pages, eligible fines, selected M) of a route (tao_stream.py:29-37).
TAO_SCHED void routed_counts(const tao_stream_cfg& c, int64_t completed, int64_t pending,
                             int64_t* coarse_out, int64_t* eligible_out,
                             int64_t* selected_out) {
  const int64_t g = c.coarse_group;
  const int64_t cb = budget(c, g * completed);
  int64_t coarse = (2 * cb + g - 1) / g;
  if (coarse > completed) coarse = completed;
  const int64_t eligible = g * coarse + pending;
  int64_t sel = budget(c, g * completed + pending);
  if (sel > eligible) sel = eligible;
  *coarse_out = coarse;
  *eligible_out = eligible;
  *selected_out = sel;
}

// Width of the next chunk from p (StreamCache.next_chunk, tao_stream.py:914-917).
inline int64_t next_chunk(const tao_stream_cfg& c, int64_t p, int64_t desired) {
  int64_t w = desired < c.fine_tokens ? desired : c.fine_tokens;
  const int64_t room = serve_limit(c) - local_len_at(c, p);
  return w < room ? w : room;
}

// The local-attention tiles of a call [pos0, pos0 + tokens): its chunks
// (next_chunk) cut into kAttnTile queries, each tile (first query row - pos0,
// count, key_start = the chunk's start - its window). emit(row, count,
// key_start) per tile, in order; the prefill plan's attention section.
constexpr int64_t kAttnTile = 256;
template <typename Emit>
inline void attention_tiles(const tao_stream_cfg& c, int64_t pos0, int64_t tokens, Emit&& emit) {
  const int64_t end = pos0 + tokens;
  for (int64_t start = pos0; start < end;) {
    const int64_t w = next_chunk(c, start, end - start);
    const int64_t key_start = start - local_len_at(c, start);
    for (int64_t qs = start; qs < start + w; qs += kAttnTile) {
      const int64_t n = start + w - qs;
      emit(qs - pos0, n < kAttnTile ? n : kAttnTile, key_start);
    }
    start += w;
  }
}

}  // namespace sched
}  // namespace tao
