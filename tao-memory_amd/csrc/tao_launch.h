// Internal launch interface between the C-ABI layer (abi.hip) and the
// kernel translation units. Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tao_memory.h"
#include "tao_common.h"

namespace tao {

constexpr int kThreads = 256;   // 4 wave64 per workgroup
constexpr int kLocalSplits = 8; // split-K factor of single-query local attention

// Workspace layout (bytes from the start of tao_state_dev::workspace):
//   [0, counters)         uint32 arrival counters: B*H per-head + 1 global
//   [parts_off, ...)      fp32 unit records [B*H][kLocalSplits + sel_cap][D + 4]
//   [tiles_off, ...)      int64 tile descriptors for multi-token kernels
struct WorkspaceLayout {
  size_t counters_off, parts_off, tiles_off, tiles_cap, total;
};

WorkspaceLayout workspace_layout(int batch, int heads, int head_dim, int sel_cap,
                                 int max_query_tokens);

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
  float* parts; uint32_t* counters;
  int B, H, keep, fine, group, fine_cap, page_cap, sel_cap;
};

// M = selected fines of the current route (0 before the first seal).
hipError_t launch_decode_step(const DecodeParams& p, int head_dim, int M, hipStream_t s);

struct StageParams {
  TokView src[5];
  bf16_t* dst;          // 5 x [B, H, D] contiguous
  int B, H, D;
};
hipError_t launch_stage_tokens(const StageParams& p, hipStream_t s);

struct AppendParams {
  TokView k, v, rk;
  bf16_t* ring_k; bf16_t* ring_v; bf16_t* ring_raw;
  int B, H, D, L, first, count;
  int64_t pos;
};
hipError_t launch_ring_append(const AppendParams& p, hipStream_t s);

struct RouteParams {
  const bf16_t* rq; int64_t rq_sb, rq_sh;
  const bf16_t* pw; const bf16_t* sw;
  int32_t* sel; int32_t* chosen; int64_t* header;
  int B, H, fine_cap, page_cap, sel_cap, chosen_cap, group;
  int completed, pending, coarse, selected;
};
hipError_t launch_route(const RouteParams& p, int head_dim, hipStream_t s);

struct WriterParams {
  TokView rk, v;                 // token operands (positions >= new_base)
  const bf16_t* ring_raw; const bf16_t* ring_v;
  bf16_t* bank; bf16_t* fine_z;
  const int64_t* starts;         // device [count] absolute start positions
  int64_t new_base;
  int B, H, L, fine_cap, first_slot, count;
};
hipError_t launch_writer(const WriterParams& p, int head_dim, hipStream_t s);

struct EpilogueParams {
  const bf16_t* fine_z; bf16_t* fine_sw; bf16_t* page_z; bf16_t* page_w;
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
};
hipError_t launch_local_attention(const AttnParams& p, int head_dim, hipStream_t s);

struct ReadParams {
  TokView rq;
  const bf16_t* bank; const bf16_t* sw; const bf16_t* pw;
  const int32_t* sel;
  const bf16_t* local;           // [B, T, H, D] contiguous
  const void* fa; const void* fb; int f_dtype;
  int64_t fa_s[3], fb_s[3];
  float gain; int coarse_on, fine_on;
  bf16_t* out; int64_t out_sb, out_st, out_sh;
  int B, H, T, first, count, selected, group, fine_cap, page_cap, sel_cap;
};
hipError_t launch_read_fuse(const ReadParams& p, int head_dim, hipStream_t s);

}  // namespace tao
