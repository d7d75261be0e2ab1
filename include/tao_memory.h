/*
 * TaoMemory attention operator: C ABI of the gfx950 (MI355X) HIP library
 * libtao_hip.so.
 *
 * The library replaces the reference's kernel layer (Triton kernels and hot
 * torch-op chains) and its regional CUDA Graph. Host code (the Python
 * tao_attention package, or any FFI) owns every buffer: the library never
 * allocates or frees caller memory. All tensors are device pointers with
 * element strides; the head dimension is contiguous. All arithmetic is on
 * bf16 storage with fp32 accumulation, except tao_full_sequence_f32 (fp32
 * operands and fp32 rounding points).
 *
 * Return convention: 0 = ok; negative = contract error (the Python host
 * raises ValueError); positive = HIP runtime error code (RuntimeError).
 * tao_last_error() returns a thread-local message for the last failure.
 *
 * Threading: stream-ordered, no internal threads; calls on one state must be
 * serialised by the caller (the reference's serial-use rule,
 * docs/graph.md:13-17).
 */
#ifndef TAO_MEMORY_H
#define TAO_MEMORY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TAO_ABI_VERSION 13

enum tao_status {
  TAO_OK = 0,
  TAO_E_SHAPE = -1,      /* unsupported head_dim / geometry / shape */
  TAO_E_CAPACITY = -2,   /* a count exceeds the state's capacity */
  TAO_E_ARGUMENT = -3,   /* null pointer or inconsistent argument */
  TAO_E_WORKSPACE = -4   /* workspace too small */
};

enum tao_dtype { TAO_BF16 = 0, TAO_FP32 = 1, TAO_FP16 = 2 };

/* Device-resident state of one request x layer (reference StreamCache +
 * LayerState, tao_stream.py:126-160, 790-834), laid out for HBM streaming:
 * a capacity-backed fine bank replaces the reference's per-seal torch.cat
 * repack (tao_stream.py:455-462) and a token ring replaces the local-window
 * concatenation (tao_stream.py:927-930, 959-969). */
typedef struct tao_state_dev {
  int32_t batch, heads, head_dim;   /* B, H, D (D in {64, 128}) */
  int32_t local_keep, fine_tokens;  /* 512, 256: ring length = their sum */
  int32_t coarse_group;             /* 8 */
  int32_t fine_cap, page_cap, sel_cap, chosen_cap;
  void* ring_k;     /* bf16 [B, L, H, D]  rotated keys, slot = position % L */
  void* ring_v;     /* bf16 [B, L, H, D]  values */
  void* ring_raw;   /* bf16 [B, L, H, D]  raw keys (writer input) */
  void* bank_c;     /* bf16 [B, H, fine_cap, D, D] fine memories */
  void* fine_z;     /* bf16 [B, H, fine_cap, D]    fine descriptors */
  void* fine_sw;    /* bf16 [B, H, fine_cap, D]    r(exp(r(z - page_z))) */
  void* page_z;     /* bf16 [B, H, page_cap, D]    completed + pending page */
  void* page_w;     /* bf16 [B, H, page_cap, D]    r(softmax over pages) */
  int32_t* sel;     /* [B, H, sel_cap]  selected fine ids, score order */
  int32_t* chosen;  /* [B, H, chosen_cap] chosen coarse pages, ascending */
  int64_t* header;  /* device [4]: position, M, reserved, reserved */
  void* fold_g;     /* fp32 [B, H, D, D]  G^T of the current route and epoch */
  void* fold_den;   /* fp32 [B, H, D]     den weights of the current route */
  /* Coarse value branch (TaoConfig.coarse_index_only = False); both null in
   * the index-only preset, both set otherwise. */
  void* page_c;     /* bf16 [B, H, page_cap, D, D] page value matrices (C^T) */
  void* coarse_g;   /* fp32 [B, H, D, D]  folded coarse read of the completed pages */
  void* workspace;  /* scratch: decode step records and the prefill plan */
  size_t workspace_bytes;
  /* Regularized association writer (TaoConfig.fine_writer =
   * "regularized_association", tao_stream.py:72-74, 463-499); all null for
   * the softmax writer. With them, every seal (tao_write_fine, tao_prefill)
   * writes C = association_matrix(u^T u, u^T v) of the block into its bank
   * slot and adds the block's statistics, in seal order, to the pending
   * sums; with page_c, a completed page's matrix is association_matrix of
   * those sums, which then restart (the index-only preset keeps summing, as
   * the reference does). */
  float* pending_gram;   /* fp32 [B, H, D, D] */
  float* pending_cross;  /* fp32 [B, H, D, D] */
  float* stats;          /* fp32 scratch [2][stats_cap * B][H][D][D] */
  int32_t stats_cap;     /* blocks per pass through the scratch (>= 1) */
  /* Feature writers (feature_mass_association, structured_gram_association;
   * tao_stream.py:56-65, 280-283, 362-367, 463-499): fine_writer selects
   * them and the read is the numerator-only mixture. A fine's z is
   * r(log mass) of its own fp32 feature mass; fine_mass[slot] holds the fp32
   * total, in seal order, of the masses of the run through that fine (the
   * reference's pending_mass after that seal), and a page or pending
   * descriptor is r(log) of it at the page's last fine. A run starts at fine
   * 0 and, with page_c (and in the full-sequence path), again at each
   * page's first fine; the streaming index-only state sums from fine 0 on,
   * as the reference clears pending_mass only when it builds page values
   * (tao_stream.py:488-497). They need stats (and stats_cap), plus
   * [stats_cap * B][H][D] floats of mass scratch after its two halves.
   * pending_gram and pending_cross (required with page_c, optional
   * index-only) hold the statistic sums of the same run: gram [B, H, D, D]
   * (feature mass) or square mass and mass [2, B, H, D] (structured), and
   * cross [B, H, D, D]; with page_c the coarse read is the mixture over
   * pages (tao_stream.py:301-305).
   * TAO_WRITER_VALUE (0): softmax descriptors (softmax and regularized). */
  int32_t fine_writer;   /* enum tao_fine_writer */
  float* fine_mass;      /* fp32 [B, H, fine_cap, D] run totals; feature writers only */
} tao_state_dev;

enum tao_fine_writer {
  TAO_WRITER_VALUE = 0,
  TAO_WRITER_FEATURE_MASS = 1,
  TAO_WRITER_STRUCTURED = 2
};

/* New-token operands: q/k/v/raw_q/raw_k, each [B, T, H, D] bf16 with
 * element strides (batch, token, head); D contiguous. */
typedef struct tao_tokens {
  const void* q; const void* k; const void* v; const void* raw_q; const void* raw_k;
  int64_t q_s[3], k_s[3], v_s[3], rq_s[3], rk_s[3];
  int32_t tokens;
} tao_tokens;

/* Caller fusion parameters: fusion_a/b [H, D, 3], both of dtype `dtype`
 * (TAO_BF16, TAO_FP32 or TAO_FP16; read in place on every call and cast to
 * bf16 round-to-nearest-even inside, fusion_pointwise.py:103-108),
 * gain = bf16(2 * alpha) (operator.py:89). */
typedef struct tao_fusion {
  const void* fusion_a; const void* fusion_b;
  int32_t dtype;
  int64_t a_s[3], b_s[3];
  float gain;
  int32_t coarse_on, fine_on;
} tao_fusion;

int tao_abi_version(void);
const char* tao_last_error(void);

/* Workspace bytes a state of this geometry needs: decode partials plus room
 * for a prefill plan of plan_words int64 (no hidden allocation). */
size_t tao_workspace_bytes(int32_t batch, int32_t heads, int32_t head_dim,
                           int32_t sel_cap, int32_t plan_words);

/* Zero a new workspace. */
int tao_workspace_init(const tao_state_dev* st, void* stream);

/* Fold the current route (replaces the per-query gather of the selected
 * fine memories in the q1 read, query_fresh_fine.py:8-75, with a
 * per-route precomputation). The read is linear in the channel weights
 * ch_m = h * w_m with w_m = pw[page(m)] * sw[m] query-independent, so for the
 * `selected` ids in st->sel under the current page weights:
 *   fold_g[e][d] = sum_m w_m[d] * C_m[d][e]     (stored as G^T, fp32)
 *   fold_den[d]  = sum_m w_m[d]
 * and one query's fine read is r(r(h.G) / r(h.den)). Call after every route
 * refresh and every seal epilogue (the stream driver and tao_prefill do). */
int tao_fold_route(const tao_state_dev* st, int32_t selected, void* stream);

/* Page value matrices of completed pages [first_page, first_page + count)
 * (replaces the page_c einsum of append_fine, tao_stream.py:486-499):
 *   page_c[g][e][d] = r(sum_s fine_sw[8g + s][d] * C^T_{8g+s}[e][d])
 * (fine_sw of a completed page is r(exp(r(z - page_z))), the reference's
 * weight). Needs st->page_c. */
int tao_page_coarse(const tao_state_dev* st, int32_t first_page, int32_t count, void* stream);

/* Fold the coarse value read over the first `completed` pages (replaces the
 * per-query coarse einsum of _read_reused, tao_stream.py:299-305): with
 * cw_p = softmax over p < completed of page_z[p],
 *   coarse_g[e][d] = sum_p cw_p[d] * page_c[p][e][d]        (fp32)
 * so one query's coarse read is r(h . coarse_g[e]). Call after every page
 * completion and after a prefill or import (the stream driver does). */
int tao_fold_coarse(const tao_state_dev* st, int32_t completed, void* stream);

/* One fused single-token decode step (replaces the memo-backed q1 region,
 * tao_stream.py:399-433, query_fresh_fine.py:52-75, the local SDPA call
 * flash_attention.py:25-29, the local concat tao_stream.py:927-930, and the
 * fusion kernels fusion_pointwise.py:95-117 / operator.py:86-94).
 * Reads the stream position from st->header[0], appends the token to the
 * ring, reads the folded route (fold_g / fold_den, see tao_fold_route) when
 * `selected` > 0 (0 before the first seal: output = local attention),
 * adds the folded coarse read (coarse_g) when fu->coarse_on, writes out
 * [B,1,H,D] (element strides out_s) and advances header[0]. One launch: its
 * workgroups meet on arrival counters in the workspace, which
 * tao_workspace_init zeroes and every step leaves at zero. */
int tao_decode_step(const tao_state_dev* st, const tao_tokens* tok,
                    const tao_fusion* fu, int32_t selected, void* out,
                    const int64_t* out_s, void* stream);

/* tao_decode_step without allocation: no reference counterpart. For callers
 * that cannot allocate device memory (code under hipGraph capture, tight
 * serving loops, harnesses that forbid hipMalloc): the same decode step,
 * arguments and results as tao_decode_step, with the step's records and
 * arrival counters in library-owned static device arrays (4 MiB, and 1024
 * counters on 128-byte lines) instead of st->workspace (which may be null).
 * Limit:
 * batch * heads <= 467 at head_dim 128, <= 531 at 64 (TAO_E_CAPACITY
 * beyond). Allocates nothing. Every call on one device shares the arrays:
 * calls that overlap on one device race and must be serialised by the
 * caller; each step leaves its counters at zero, so nothing needs clearing
 * between calls. */
int tao_decode_step_noalloc(const tao_state_dev* st, const tao_tokens* tok,
                            const tao_fusion* fu, int32_t selected, void* out,
                            const int64_t* out_s, void* stream);

/* Routing refresh from one anchor query row (replaces tao_stream.py:310-357
 * and _topk_oldest :50-53). raw_q_row: [B, H, D] view with strides rq_s
 * (batch, head). Writes st->sel / st->chosen and header[1] = M. */
int tao_route(const tao_state_dev* st, const void* raw_q_row,
              const int64_t* rq_s, int32_t completed, int32_t pending,
              int32_t coarse, int32_t selected, void* stream);

/* Softmax fine writer for `count` blocks (replaces _seal, tao_stream.py:
 * 56-77, and the packed-bank append :455-462). Block i covers absolute
 * positions [start_pos[i], start_pos[i] + fine_tokens) read from the ring
 * (positions < new_base) or from the token operands (>= new_base); its
 * z / C go to fine slot first_slot + i. start_pos: device int64 [count]. */
int tao_write_fine(const tao_state_dev* st, const tao_tokens* tok,
                   int64_t new_base, const int64_t* start_pos,
                   int32_t first_slot, int32_t count, void* stream);

/* Page bookkeeping after sealing fine `slot` (replaces append_fine's
 * page summary tao_stream.py:477-501, the pending summary :277-290 and the
 * seal-epoch memo _prepare_q1_page_memo :399-416): page descriptor of the
 * slot's group, segment weights of the group's fines, page weights over the
 * `pages` current pages. recompute = 0 keeps the group's page descriptor
 * already in page_z (snapshot import) instead of recomputing it. */
int tao_seal_epilogue(const tao_state_dev* st, int32_t slot, int32_t pages,
                      int32_t recompute, void* stream);

/* Exact local attention with the suffix causal mask (replaces
 * flash_attn_func, flash_attention.py:16-37, and the local-window concat,
 * tao_stream.py:927-930). Query row r of tok.q sits at absolute position
 * qpos0 + r; key row j of tok.k / tok.v at kpos0 + j, and keys older than
 * kpos0 come from the ring. tiles: device int64 [n_tiles][3] = (first query
 * row, count <= 256, key_start): the tile's queries see keys from key_start
 * up to their own position. local: bf16 [B, tok.tokens, H, D] contiguous. */
int tao_local_attention(const tao_state_dev* st, const tao_tokens* tok,
                        int64_t qpos0, int64_t kpos0, const int64_t* tiles,
                        int32_t n_tiles, void* local, void* stream);

/* Epoch pools of one prefill call (caller-allocated):
 *   pw_pool  bf16 [epochs][B][H][pool_pcap][D]  page weights per seal epoch
 *   psw_pool bf16 [epochs][B][H][coarse_group][D] pending segment weights
 *   sel_pool int32 [sel_slots][B][H][sel_cap]   selected ids per route turn
 *   coarse_pool bf16 [coarse_count][B][H][D][D] folded coarse reads (G^T)
 *     for completed = coarse_first + i (coarse value branch only; else null)
 *   qsel     uint32 [B][T][H][qsel_words]      per-query selections as
 *     bitmasks over fine ids (plans with TAO_PLAN_QUERY_ROUTES = 1 only)
 * Slot 0 of sel_pool receives the state's route at call start. */
typedef struct tao_prefill_pools {
  void* pw_pool; void* psw_pool; int32_t* sel_pool;
  int32_t pool_pcap, epochs, sel_slots;
  void* coarse_pool;
  int32_t coarse_first, coarse_count;
  uint32_t* qsel;
  int32_t qsel_words;
  /* Optional forward saves for the full-sequence backward (null = skip):
   * local_lse fp32 [B][T][H] log2-sum-exp of each query's local scores
   * (scale 1/sqrt(D) * log2 e); coarse_out / fine_out bf16 [B][T][H][D]
   * the coarse and fine heads before the fusion (history queries only);
   * den_out fp32 [B][T][H] the fine read's denominator. */
  float* local_lse;
  void* coarse_out;
  void* fine_out;
  float* den_out;
  /* Nonzero: the caller has written the fine value matrices (bank_c) of the
   * blocks this call seals and the page value matrices (page_c) of the pages
   * it completes, as the non-softmax writers do (tao_stream.py:56-77,
   * :486-499, association_writer.py); the writer then computes only fine_z
   * and the page pass only the page descriptors and weights. */
  int32_t external_values;
} tao_prefill_pools;

/* Layout of the int64 prefill plan (all indices are token offsets in tok
 * unless noted). Header of TAO_PLAN_HEADER words, then the arrays. */
#define TAO_PLAN_HEADER 16
enum tao_plan_field {
  TAO_PLAN_POS0 = 0,        /* absolute position of token 0 */
  TAO_PLAN_ATTN_TILES = 1,  /* n, then n x {first, count <= 256, key_start} */
  TAO_PLAN_WRITES = 2,      /* n, then n block start positions */
  TAO_PLAN_FIRST_SLOT = 3,  /* fine slot of the first written block */
  TAO_PLAN_FIRST_PAGE = 4,  /* first page completed by this call */
  TAO_PLAN_PAGES = 5,       /* number of pages completed by this call */
  TAO_PLAN_FIRST_EPOCH = 6, /* first seal epoch (visible fines) read */
  TAO_PLAN_EPOCHS = 7,      /* epochs, the last one is published */
  TAO_PLAN_TURNS = 8,       /* n, then n x {anchor, epoch - first_epoch,
                               completed, pending, coarse, selected,
                               sel slot, publish} */
  TAO_PLAN_READ_TILES = 9,  /* n, then n x {first, count <= 32, sel slot,
                               selected, epoch - first_epoch, sw split,
                               fine_on, completed pages} */
  TAO_PLAN_RING_FIRST = 10, /* ring append: first token, count, position */
  TAO_PLAN_RING_COUNT = 11,
  TAO_PLAN_RING_POS = 12,
  TAO_PLAN_QUERY_ROUTES = 13 /* 1: every history query routes itself (no
                                turns; read tile field 2 holds the coarse
                                page count of its epoch, selections go to
                                pools.qsel) */
};

/* Batched prefill of tok.tokens new tokens (replaces the chunk loop of
 * tao_attention_prefill, operator.py:100-127, with StreamCache.process,
 * tao_stream.py:919-979, for every chunk): local attention for all chunks,
 * the writer for every seal, page/epoch bookkeeping, routes for every
 * refresh turn, selected read + fusion for every query, ring append. The
 * plan is validated on the host and copied into the workspace. local:
 * bf16 [B, T, H, D] scratch for the local attention output. */
int tao_prefill(const tao_state_dev* st, const tao_tokens* tok,
                const tao_fusion* fu, const int64_t* plan, int64_t plan_len,
                const tao_prefill_pools* pools, void* local, void* out,
                const int64_t* out_s, void* stream);

/* Copy `count` tokens starting at token `first` of tok into the ring at
 * absolute positions [pos, pos + count) (keys, values, raw keys). */
int tao_ring_append(const tao_state_dev* st, const tao_tokens* tok,
                    int32_t first, int32_t count, int64_t pos, void* stream);

/* hipGraph of the decode step (the captured region of HistoryRegionGraph,
 * history_region_graph.py:95-113). The graph holds one node, the decode step
 * with its cursor read on the device, writing out_stage (bf16 [B,1,H,D]);
 * it is instantiated twice and tao_graph_launch alternates between the two
 * executable graphs, pointing the step at the call's operands
 * (hipGraphExecKernelNodeSetParams) before each hipGraphLaunch. The
 * reference copies its operands into static inputs instead (raw_input);
 * reading them in place saves that copy and the graph edge after it. The
 * stream driver ends the epoch at each refresh and seal, as the reference
 * does. staging is unused (may be NULL). */
int tao_graph_create(const tao_state_dev* st, const tao_fusion* fu,
                     int32_t selected, void* staging, void* out_stage,
                     void* stream, void** graph_out);
int tao_graph_launch(void* graph, const tao_tokens* tok, void* stream);
int tao_graph_destroy(void* graph);

/* Diagnostic clock stamps of eager decode steps; no counterpart in the
 * reference (it is for latency timelines of the single-launch step). While
 * on, decode step i with a host cursor writes frame i % frames of buf
 * (uint64, frame_words words per frame): per workgroup 8 words at
 * blockIdx * 8, the device's 100 MHz clock (s_memrealtime) at entry, after
 * a local unit's scores, after its record stores issued, after their
 * acknowledgement barrier, after its arrival count, after the merge (the
 * head's last arrival only, else 0), then (unit << 32 | batch * H + head)
 * and (XCC << 32 | __smid()). A launch whose grid does not fit a frame records nothing.
 * buf NULL turns it off; the count restarts at every call. Host state of
 * the library, not thread-safe. */
int tao_step_stamps(void* buf, int64_t frames, int64_t frame_words);
int64_t tao_step_stamps_count(void);

/* Streaming geometry of one request x layer (reference TaoConfig fields,
 * config.py:7-19, and the layer index that staggers route refreshes). */
typedef struct tao_stream_cfg {
  int32_t layer, local_keep, fine_tokens, coarse_group, route_period, layer_stagger;
  int32_t budget_root_scale, budget_offset;
  int32_t use_graph;   /* decode-graph epochs (history_region_graph.py:66-113):
                          0 off; 1 replay by direct dispatch of the recorded
                          step; 2 replay a hipGraph (tao_graph_create) */
} tao_stream_cfg;

/* Plan of one tao_prefill call for tokens [pos0, pos0 + tokens) of a
 * request x layer (replaces the host chunk loop of tao_attention_prefill,
 * operator.py:100-127, and the turn split of _read_progressive,
 * tao_stream.py:196-227). route_coarse / route_size: the state's current
 * route; outputs = 0 plans a state-only advance (no attention or reads; the
 * last refresh turn is routed alone). With plan == NULL only info is filled
 * (a size query). info (int64[10]) receives: plan length, epochs, turns,
 * route coarse and route size after the call, page capacity of the epoch
 * pools, chunks that read history, chunks, and the coarse pool range
 * (first completed-page count >= 1 read, number of counts). Host code only. */
int tao_prefill_plan(const tao_stream_cfg* cfg, int64_t pos0, int64_t tokens,
                     int32_t route_coarse, int32_t route_size, int32_t outputs,
                     int64_t* plan, int64_t plan_cap, int64_t* info);

/* Local attention of a call whose window holds only the call's own tokens,
 * without a state (the same kernel and tiles as tao_prefill's local
 * attention), so that a caller can start it before it allocates a new
 * state: the reference's first chunks of a prompt (flash_attn_func,
 * flash_attention.py:16-37, over the window of tao_stream.py:927-930 at
 * position 0). The tiles are those of the call's tao_prefill_plan attention
 * section (the schedule's chunks of cfg from pos0 over tok.tokens); each
 * must lie in the call's tokens (key_start >= pos0: no key from a ring,
 * which holds for pos0 = 0) and is written to tiles_dev (device int64,
 * tiles_cap words, at least 3 per tile) on the stream. local: bf16
 * [B, tok.tokens, H, D] contiguous. The caller then passes tao_prefill the
 * plan without its attention section and this local output. */
int tao_prompt_attention(const tao_stream_cfg* cfg, int32_t batch, int32_t heads,
                         int32_t head_dim, const tao_tokens* tok, int64_t pos0,
                         void* tiles_dev, int64_t tiles_cap, void* local, void* stream);

/* Plan of the full-sequence read of tokens [0, tokens) (replaces the host
 * tiling of read_training, tao_stream.py:668-757, and of
 * _local_training_corrected_4k, :760-787, behind tao_attention,
 * operator.py:40-52), executed by tao_prefill on a fresh state: tile t of
 * fine_tokens queries attends suffix-causally to keys from
 * max(0, t * fine_tokens - local_keep), reads the first
 * max(0, t - local_keep / fine_tokens) sealed fines, and every one of its
 * queries routes itself (TAO_PLAN_QUERY_ROUTES). Only the visible blocks are
 * written; nothing is appended to the ring. info (int64[12]): the ten
 * tao_prefill_plan fields (turns = 0), then the fines written and
 * qsel_words, the bitmask words per query. Host code only. */
int tao_train_plan(const tao_stream_cfg* cfg, int64_t tokens, int64_t* plan,
                   int64_t plan_cap, int64_t* info);

/* Backward of the full-sequence read (replaces the reference's autograd
 * through tao_attention: _fuse_training, operator.py:21-38; the local SDPA,
 * tao_stream.py:760-787; _SelectedRead.backward, selected_read.py:175-187;
 * the page / segment softmaxes and logsumexps, tao_stream.py:530-665; the
 * writers, tao_stream.py:80-123: softmax, regularized association through
 * its solve, and the feature writers through their mixture reads
 * (feature_read_coefficients and selected_fine_numerator,
 * association_writer.py:46-53, indirect_fine.py:65-120), log-mass
 * descriptors and the solve or structured closed form,
 * structured_writer.py:16-34). st, tok, fu and pools are the
 * forward's tao_prefill arguments (same buffers, unchanged since), and the
 * forward was run with pools.local_lse / coarse_out / fine_out / den_out set
 * (local: its local-attention scratch). grad: upstream gradient bf16
 * [B, T, H, D] with element strides grad_s (batch, token, head). Outputs:
 * bf16 [B, T, H, D] contiguous dq, dk, dv, draw_q, draw_k; dfusion_a /
 * dfusion_b fp32 [H, D, 3], accumulated (zero them first). No gradient for
 * alpha (the reference builds the gain from a Python float, operator.py:34).
 * workspace: tao_train_bwd_workspace_bytes(...) bytes of device memory. */
typedef struct tao_train_bwd {
  const void* grad; int64_t grad_s[3];
  const void* local; const float* local_lse;
  const void* coarse_out; const void* fine_out; const float* den_out;
  void* dq; void* dk; void* dv; void* draw_q; void* draw_k;
  float* dfusion_a; float* dfusion_b;
  void* workspace; size_t workspace_bytes;
  /* Optional (null = skip): the memory adjoints before the writer,
   * d fine_z fp32 [B][H][fines][D] and d C^T fp32 [B][H][fines][D][D]
   * ([e][d], the bank's layout), for callers that inspect them (feature
   * writers: d fine_z of the fine mixture read; the page descriptors' share
   * goes to the masses directly). */
  float* dz_out; float* dc_out;
  /* Optional (null = skip): fp32 [1] receives d out / d alpha . grad through
   * gain = 2 alpha (no reference counterpart: the reference takes alpha as a
   * Python float, operator.py:34). */
  float* dalpha_out;
  /* Optional: bf16 [B, T, H, D] contiguous. Non-null when the forward's local
   * attention came from a caller plugin (tao_attention's local_flash,
   * operator.py:42-47, tao_stream.py:760-787): it receives d out / d local,
   * the local-attention adjoint is skipped (the caller differentiates its
   * plugin), local_lse, dq and dk may be null, and dv holds only the
   * writer's share. */
  void* dlocal_out;
} tao_train_bwd;

/* Workspace bytes of tao_train_backward for a full-sequence read of `tokens`
 * tokens whose plan wrote `fines` fines (tao_train_plan info[10]). */
size_t tao_train_bwd_workspace_bytes(const tao_state_dev* st, int64_t tokens, int32_t fines,
                                     const tao_prefill_pools* pools);

int tao_train_backward(const tao_state_dev* st, const tao_tokens* tok, const tao_fusion* fu,
                       const tao_prefill_pools* pools, const tao_train_bwd* args,
                       void* stream);

/* fp32 full-sequence read: tao_attention on fp32 operands (replaces the
 * reference's read_training + _fuse_training at fp32, operator.py:21-54,
 * tao_stream.py:80-123, 530-787). tok: fp32 [B, T, H, D] views (element
 * strides, channel stride 1; tokens = T). fu: fusion parameters of any
 * tao_dtype; gain = fp32(2 alpha). out: fp32 [B, T, H, D]. cfg: the
 * geometry (512/256/8) and the budget; layer, route_period, layer_stagger
 * and use_graph are unused. coarse_values: 0 for coarse_index_only.
 * Every rounding point of the bf16 contract rounds to fp32, and routing
 * sums keep the bf16 path's orders, so routes are reproducible bit for
 * bit. Forward only. At most 64 pages and 256 route candidates per query
 * (TAO_E_CAPACITY beyond). sel_out (optional, int32 [B, T, H, sel_cap]):
 * each query's selected fine ids in score order, -1 padded (-1 throughout
 * before first_fine). workspace: tao_full_sequence_f32_workspace_bytes()
 * bytes of device memory, fully written before it is read. */
size_t tao_full_sequence_f32_workspace_bytes(int32_t batch, int32_t heads, int32_t head_dim,
                                             int64_t tokens, int32_t coarse_values);
int tao_full_sequence_f32(const tao_stream_cfg* cfg, const tao_tokens* tok, const tao_fusion* fu,
                          int32_t batch, int32_t heads, int32_t head_dim, int32_t coarse_values,
                          void* out, const int64_t* out_s, int32_t* sel_out, int32_t sel_cap,
                          void* workspace, size_t workspace_bytes, void* stream);

/* tao_full_sequence_f32 with the local attention supplied by the caller
 * (the reference's read_training called with a local_flash plugin on fp32
 * operands, operator.py:40-52, tao_stream.py:760-787): local is fp32
 * [B, T, H, D] contiguous, read only; the read, routes and fusion are those
 * of tao_full_sequence_f32. */
int tao_full_sequence_f32_local(const tao_stream_cfg* cfg, const tao_tokens* tok,
                                const tao_fusion* fu, int32_t batch, int32_t heads,
                                int32_t head_dim, int32_t coarse_values, const void* local,
                                void* out, const int64_t* out_s, int32_t* sel_out,
                                int32_t sel_cap, void* workspace, size_t workspace_bytes,
                                void* stream);

/* Numerics self-test (no reference counterpart): y[i] = the library's
 * bf16(correctly rounded fp32 exp(x[i])) (op 0) or log (op 1) for n bf16
 * device inputs, the functions every writer and page kernel uses; op 2 / 3:
 * x holds n fp32 values (n a multiple of 64), y[g] = the fp32 fold sum of
 * x[64 g .. 64 g + 63] as the routing kernels compute it (op 2: DPP fold on
 * the bit-reversed lane layout; op 3: shuffle butterfly). */
int tao_numerics_selftest(int32_t op, const void* x, void* y, int64_t n, void* stream);

/* Native per-token driver (replaces the Python control flow of one decode
 * call: operator.py:130-138, tao_stream.py:196-249 and 919-969,
 * history_region_graph.py:66-113). It keeps the cursor and the current route
 * size; out_stage (bf16 [B,1,H,D]) is the caller's graph output buffer (may
 * be null when use_graph is 0); staging is unused (may be NULL). */
int tao_stream_open(const tao_state_dev* st, const tao_stream_cfg* cfg, int64_t position,
                    int32_t route_coarse, int32_t route_size, void* staging,
                    void* out_stage, void** handle);
/* Re-point the driver after the host grew buffers, prefilled or imported.
 * An open graph epoch sees the advance as the reference's prefill does: its
 * route refreshes copy ids (or end the epoch on a new route size), a seal
 * ends it; moved buffers end it as an epoch change. */
int tao_stream_sync(void* handle, const tao_state_dev* st, int64_t position,
                    int32_t route_coarse, int32_t route_size);
/* One new token: route refresh on turn positions, the decode step, and the
 * seal when the local window fills. With use_graph the non-refresh steps of
 * one epoch (same state version, route size and fusion parameters) follow
 * HistoryRegionGraph.run (history_region_graph.py:66-113): three eager
 * steps into out, then one capture and replays whose heads land in
 * out_stage; a refresh step copies its route into the epoch (or ends it
 * when the route size changed) and a seal ends it. out is always required.
 * info (int64[7]) receives: position after the call, route coarse count,
 * route size, refreshed, sealed, heads in out_stage (replay), captured. */
int tao_stream_decode(void* handle, const tao_tokens* tok, const tao_fusion* fu, void* out,
                      const int64_t* out_s, void* stream, int64_t* info);
/* Device-cursor steps for a caller's whole-step graph across layers (the
 * caller-side multi-layer decode of docs/benchmarks.md:15, 89-94; no
 * reference entry point: the reference captures one layer's region only,
 * history_region_graph.py:95-113).
 * tao_stream_plan_step: the driver's next token. info (int64[7]) receives
 *   its position, whether a route refresh is due before its step, whether a
 *   seal is due after it, the route size its step reads, the fine and
 *   coarse presence flags of its fusion, and whether a refresh in its state
 *   version keeps the current route (coarse count and size unchanged).
 * tao_stream_graph_step: launches the next token's work with the cursor
 *   read on the device (header[0], advanced by the step), so a caller may
 *   capture it in a hipGraph and replay it for successive tokens of one
 *   state version: when refreshes keep the route (info[6]), the route
 *   refresh and fold kernels first, each exiting on the device unless the
 *   cursor is a refresh turn of the stream's layer, then the decode step.
 *   A captured launch replays correctly for every token of its state
 *   version that has no seal after it and whose refresh, if any, keeps the
 *   route; the caller checks with tao_stream_plan_step (no seal, and no
 *   refresh or info[6]) and runs other tokens through tao_stream_decode.
 *   Fails for a token that is not such a token. The host cursor does not
 *   move.
 * tao_stream_advance: moves the host cursor over `count` such tokens that
 *   ran as device-cursor steps (fails if one of them is not). */
int tao_stream_plan_step(void* handle, int64_t* info);
int tao_stream_graph_step(void* handle, const tao_tokens* tok, const tao_fusion* fu, void* out,
                          const int64_t* out_s, void* stream);
int tao_stream_advance(void* handle, int64_t count);
/* Batched decode of `count` independent requests of one layer (no reference
 * counterpart: the reference decodes one request per call; this serves
 * many streams, BASELINE config 5, with one decode step launch pair).
 * handles: the requests' stream drivers (tao_stream_open) over states of
 * batch 1 that share heads, head width, geometry and coarse branch. table:
 * caller device memory of tao_batch_table_bytes(count) bytes, filled by
 * tao_batch_open and refreshed by tao_batch_sync after any member's buffers
 * moved (tao_stream_sync first). One tao_batch_decode call = one new token
 * per request: each request's route refresh and seal as its own cursor
 * requires (tao_stream_decode's rules, eager), then one decode step for all
 * requests. tok / out: [count, 1, H, D] views, request r = batch row r.
 * info (int64[4 * count]): per request refreshed, sealed, route coarse
 * count, route size. The results equal one tao_stream_decode per request. */
size_t tao_batch_table_bytes(int32_t count);
int tao_batch_open(void* const* handles, int32_t count, void* table, size_t table_bytes,
                   void* stream, void** batch);
int tao_batch_sync(void* batch, void* stream);
int tao_batch_decode(void* batch, const tao_tokens* tok, const tao_fusion* fu, void* out,
                     const int64_t* out_s, void* stream, int64_t* info);
int tao_batch_close(void* batch);

/* Why a decode-graph epoch ended (HistoryRegionGraph.invalidate callers:
 * history_region_graph.py:60, 78; tao_stream.py:406, 445, 841, and this
 * library's buffer growth). */
enum tao_graph_reason {
  TAO_GRAPH_SEAL = 0,
  TAO_GRAPH_SELECTED_SHAPE = 1,
  TAO_GRAPH_EPOCH_CHANGE = 2,
  TAO_GRAPH_MEMO_REPLACE = 3,
  TAO_GRAPH_REQUEST_END = 4,
  TAO_GRAPH_RESET = 5,
  TAO_GRAPH_CAPACITY = 6,
  TAO_GRAPH_REASONS = 7
};
/* Epoch counters of the driver (HistoryRegionGraph.counts and observation(),
 * history_region_graph.py:19-37), as int64 words at these indices; last
 * action: 0 uninitialized, 1 eager_warm, 2 capture_replay, 3 replay,
 * 4 route_copy, 5 invalidate (last reason in TAO_GS_LAST_REASON). */
enum tao_graph_stat {
  TAO_GS_EPOCHS = 0,
  TAO_GS_EAGER_WARM = 1,
  TAO_GS_CAPTURES = 2,
  TAO_GS_REPLAYS = 3,
  TAO_GS_ID_COPIES = 4,
  TAO_GS_INVALIDATIONS = 5,
  TAO_GS_ACTIVE_GRAPH = 6,      /* a captured step exists */
  TAO_GS_ACTIVE_EPOCH = 7,      /* an epoch is open (its staging is bound) */
  TAO_GS_EPOCH_VERSION = 8,     /* state version of the open epoch, or -1 */
  TAO_GS_WARM = 9,              /* eager steps of the open epoch */
  TAO_GS_LAST_ACTION = 10,
  TAO_GS_LAST_REASON = 11,
  TAO_GS_REASON0 = 12,          /* + tao_graph_reason: invalidations by reason */
  TAO_GRAPH_STATS = 12 + TAO_GRAPH_REASONS
};
/* End the open epoch for `reason` (counted once, as
 * HistoryRegionGraph.invalidate) and destroy its captured step; the
 * semantic state is untouched. No-op when no epoch is open. */
int tao_stream_invalidate(void* handle, int32_t reason);
/* Copy min(n, TAO_GRAPH_STATS) epoch counters into stats. */
int tao_stream_graph_stats(void* handle, int64_t* stats, int32_t n);
/* tao_stream_invalidate(handle, TAO_GRAPH_REQUEST_END). */
int tao_stream_release(void* handle);
int tao_stream_close(void* handle);

/* ---- Non-preset fine writers (TaoConfig.fine_writer other than "softmax")
 * and the channel-given selected read. Plain operators on caller buffers,
 * stream-ordered, no allocation. Statistics and matrices are [.., D, D]
 * row-major with rows d (feature channel) and columns e (value channel), as
 * the reference's. */
enum tao_stats_mode { TAO_STATS_ASSOCIATION = 0, TAO_STATS_STRUCTURED = 1 };

/* Simplex-feature statistics of `blocks` independent token blocks; k, v bf16
 * [blocks, tokens, H, D] with element strides (block, token, head), D
 * contiguous; u = bf16(softmax_D(fp32 k)). Outputs fp32, contiguous:
 *   TAO_STATS_ASSOCIATION (association_statistics,
 *     association_writer.py:11-18): gram [blocks, H, D, D] = u^T u,
 *     cross [blocks, H, D, D] = u^T v, mass [blocks, H, D] = sum_t u
 *     (nullable: with_mass=False);
 *   TAO_STATS_STRUCTURED (structured_statistics, structured_writer.py:5-13):
 *     gram receives square_mass [blocks, H, D] = sum_t u^2, cross, mass. */
int tao_writer_statistics(const void* k, const int64_t* k_s, const void* v, const int64_t* v_s,
                          int32_t blocks, int32_t tokens, int32_t heads, int32_t head_dim,
                          int32_t mode, float* gram, float* cross, float* mass, void* stream);

/* association_matrix (association_writer.py:21-32) of `count` independent
 * fp32 pairs [count, D, D]: out = bf16(X), (gram + trace(gram)/D I) X = cross,
 * by a Cholesky factor. info (nullable, int32 [count]) receives 0, or j + 1
 * when pivot j of the factor is not positive; the reference raises there
 * (torch.linalg.cholesky) unless unchecked. */
int tao_association_matrix(const float* gram, const float* cross, int32_t count, int32_t head_dim,
                           void* out, int32_t* info, void* stream);

/* structured_matrix (structured_writer.py:16-34): the analytic inverse of
 * diag(var + ridge) - var var^T / sum(var) + mass mass^T / tokens applied to
 * cross (var = max(square_mass - mass^2 / tokens, 0), ridge = mean
 * square_mass), fp32 in [count, D] / [count, D, D], bf16 out [count, D, D]. */
int tao_structured_matrix(const float* square_mass, const float* cross, const float* mass,
                          int32_t count, int32_t head_dim, float tokens, void* out, void* stream);

/* chronological_sum (association_writer.py:35-40): out[o][i] = fp32 sum over
 * f in order of x[o][f][i], x contiguous [outer, fines, inner]. */
int tao_chronological_sum(const float* statistics, int64_t outer, int32_t fines, int64_t inner,
                          float* out, void* stream);

/* feature_read_coefficients (association_writer.py:43-53): h bf16
 * [B, T, H, D] (strides h_s: b, t, h); read_z bf16 broadcastable to
 * [B, T, H, P, D] (strides z_s: b, t, h, p; 0 on a broadcast axis);
 * out bf16 [B, T, H, P, D] contiguous =
 * bf16(mass_p / sum_p mass_p * h), mass_p = sum_d h[d] exp(z_p[d]). */
int tao_feature_read_coefficients(const void* h, const int64_t* h_s, const void* read_z,
                                  const int64_t* z_s, int32_t batch, int32_t tokens,
                                  int32_t heads, int32_t pages, int32_t head_dim, void* out,
                                  void* stream);

/* selected_fine_numerator (indirect_fine.py:123-133, _SelectedContraction
 * :65-120): channel bf16 [B, Q, H, M, D], selected_id int64 [B, Q, H, M],
 * fine_c bf16 [BB, H, S, D, D] (batch b reads bank b % BB), all contiguous;
 * out bf16 [B, Q, H, D] = bf16(sum_m channel_m . C[id_m]). M <= 64,
 * S <= 4096; ids outside [0, S) contribute nothing. */
int tao_selected_numerator(const void* channel, const int64_t* selected_id, const void* fine_c,
                           int32_t batch, int32_t queries, int32_t heads, int32_t selected,
                           int32_t bank_batch, int32_t fines, int32_t head_dim, void* out,
                           void* stream);
/* Its backward (_SelectedContraction.backward, indirect_fine.py:101-120):
 * grad bf16 [B, Q, H, D]; grad_channel (nullable) bf16 [B, Q, H, M, D] =
 * bf16(grad . C[id_m]^T) (_grouped_grad_a :172-195); grad_fine_c (nullable)
 * bf16 [BB, H, S, D, D] = bf16(sum over b % BB == bb of bf16(per-batch
 * sum of channel^T grad over the pairs selecting each fine))
 * (_shared_grad_c :198-227). Every element of both outputs is written. */
int tao_selected_numerator_backward(const void* channel, const int64_t* selected_id,
                                    const void* fine_c, const void* grad, int32_t batch,
                                    int32_t queries, int32_t heads, int32_t selected,
                                    int32_t bank_batch, int32_t fines, int32_t head_dim,
                                    void* grad_channel, void* grad_fine_c, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TAO_MEMORY_H */
