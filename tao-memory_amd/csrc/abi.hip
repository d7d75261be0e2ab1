// C ABI of libtao_hip.so (declared in include/tao_memory.h).
//
// Validates shapes and capacities on the host before any launch (contract
// errors return negative codes, HIP failures their positive hipError_t),
// translates the plain-pointer structs into kernel parameter blocks and owns
// the only library-side resources: hipGraphExec objects of the decode step.
#include <algorithm>
#include <cstdlib>
#include <string>
#include <vector>

#include "schedule.h"
#include "tao_launch.h"

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int check_hip(hipError_t e, const char* where) {
  if (e == hipSuccess) return TAO_OK;
  g_error = std::string(where) + ": " + hipGetErrorString(e);
  return (int)e;
}

// Regularized association writer (state buffers set, tao_memory.h).
// Feature writers (fine_writer TAO_WRITER_FEATURE_MASS / _STRUCTURED).
bool feature_writer(const tao_state_dev* st) { return st->fine_writer != TAO_WRITER_VALUE; }

bool assoc_writer(const tao_state_dev* st) {
  return st->pending_gram != nullptr && !feature_writer(st);
}

int check_assoc(const tao_state_dev* st) {
  if (feature_writer(st)) return TAO_OK;   // check_feature covers its buffers
  const bool any = st->pending_gram || st->pending_cross || st->stats;
  if (any && (!st->pending_gram || !st->pending_cross || !st->stats || st->stats_cap < 1))
    return fail(TAO_E_ARGUMENT,
                "the regularized writer needs pending_gram, pending_cross and stats (stats_cap >= 1)");
  return TAO_OK;
}

int check_feature(const tao_state_dev* st) {
  if (st->fine_writer != TAO_WRITER_VALUE && st->fine_writer != TAO_WRITER_FEATURE_MASS &&
      st->fine_writer != TAO_WRITER_STRUCTURED)
    return fail(TAO_E_ARGUMENT, "unknown fine_writer");
  if (!feature_writer(st)) {
    if (st->fine_mass) return fail(TAO_E_ARGUMENT, "fine_mass is set without a feature writer");
    return TAO_OK;
  }
  if (!st->fine_mass || !st->stats || st->stats_cap < 1)
    return fail(TAO_E_ARGUMENT, "a feature writer needs fine_mass and stats (stats_cap >= 1)");
  if ((st->pending_gram != nullptr) != (st->pending_cross != nullptr) ||
      (st->page_c != nullptr && st->pending_gram == nullptr))
    return fail(TAO_E_ARGUMENT,
                "a feature writer's pending sums are both set or both null, and set with page "
                "values: pending_gram ([B, H, D, D], or [2, B, H, D] square mass and mass for "
                "the structured writer) and pending_cross");
  return TAO_OK;
}

int check_state(const tao_state_dev* st, bool need_workspace = true) {
  if (!st) return fail(TAO_E_ARGUMENT, "null state");
  if (st->head_dim != 64 && st->head_dim != 128)
    return fail(TAO_E_SHAPE, "head_dim must be 64 or 128 on the HIP path");
  if (st->local_keep != 512 || st->fine_tokens != 256)
    return fail(TAO_E_SHAPE, "HIP kernels implement local_keep=512, fine_tokens=256");
  if (st->batch <= 0 || st->heads <= 0 || st->coarse_group <= 0)
    return fail(TAO_E_SHAPE, "batch, heads and coarse_group must be positive");
  if (!st->ring_k || !st->ring_v || !st->ring_raw || !st->bank_c || !st->fine_z ||
      !st->fine_sw || !st->page_z || !st->page_w || !st->sel || !st->chosen ||
      !st->header || !st->fold_g || !st->fold_den || (need_workspace && !st->workspace))
    return fail(TAO_E_ARGUMENT, "state has a null device buffer");
  if ((st->page_c == nullptr) != (st->coarse_g == nullptr))
    return fail(TAO_E_ARGUMENT, "page_c and coarse_g must be both set or both null");
  if (st->sel_cap > 512) return fail(TAO_E_CAPACITY, "sel_cap above 512");
  if (st->coarse_group != 8) return fail(TAO_E_SHAPE, "HIP kernels implement coarse_group=8");
  if (int rc = check_assoc(st)) return rc;
  if (int rc = check_feature(st)) return rc;
  const tao::WorkspaceLayout lay =
      tao::workspace_layout(st->batch, st->heads, st->head_dim, st->sel_cap, 0);
  if (need_workspace && st->workspace_bytes < lay.plan_off)
    return fail(TAO_E_WORKSPACE, "workspace smaller than tao_workspace_bytes()");
  return TAO_OK;
}

size_t plan_capacity(const tao_state_dev* st) {
  const tao::WorkspaceLayout lay =
      tao::workspace_layout(st->batch, st->heads, st->head_dim, st->sel_cap, 0);
  return (st->workspace_bytes - lay.plan_off) / sizeof(int64_t);
}

int64_t* plan_of(const tao_state_dev* st) {
  const tao::WorkspaceLayout lay =
      tao::workspace_layout(st->batch, st->heads, st->head_dim, st->sel_cap, 0);
  return (int64_t*)((char*)st->workspace + lay.plan_off);
}

tao::TokView view(const void* p, const int64_t* s) {
  tao::TokView v;
  v.p = (const bf16_t*)p;
  v.sb = s[0];
  v.st = s[1];
  v.sh = s[2];
  return v;
}

float* parts_of(const tao_state_dev* st) {
  const tao::WorkspaceLayout lay =
      tao::workspace_layout(st->batch, st->heads, st->head_dim, st->sel_cap, 0);
  return (float*)((char*)st->workspace + lay.parts_off);
}

tao::DecodeParams decode_params(const tao_state_dev* st, const tao_tokens* tok,
                                const tao_fusion* fu, void* out, const int64_t* out_s) {
  tao::DecodeParams p{};
  p.q = view(tok->q, tok->q_s);
  p.k = view(tok->k, tok->k_s);
  p.v = view(tok->v, tok->v_s);
  p.rq = view(tok->raw_q, tok->rq_s);
  p.rk = view(tok->raw_k, tok->rk_s);
  p.ring_k = (bf16_t*)st->ring_k;
  p.ring_v = (bf16_t*)st->ring_v;
  p.ring_raw = (bf16_t*)st->ring_raw;
  p.bank = (const bf16_t*)st->bank_c;
  p.sw = (const bf16_t*)st->fine_sw;
  p.pw = (const bf16_t*)st->page_w;
  p.sel = st->sel;
  p.header = st->header;
  p.fa = fu->fusion_a;
  p.fb = fu->fusion_b;
  p.f_dtype = fu->dtype;
  for (int i = 0; i < 3; ++i) { p.fa_s[i] = fu->a_s[i]; p.fb_s[i] = fu->b_s[i]; }
  p.gain = fu->gain;
  p.out = (bf16_t*)out;
  p.out_sb = out_s[0];
  p.out_sh = out_s[2];
  p.parts = st->workspace ? parts_of(st) : nullptr;
  p.counters = nullptr;
  if (st->workspace) {
    const tao::WorkspaceLayout lay =
        tao::workspace_layout(st->batch, st->heads, st->head_dim, st->sel_cap, 0);
    p.counters = (unsigned*)((char*)st->workspace + lay.count_off);
  }
  p.fold_g = (const float*)st->fold_g;
  p.fold_den = (const float*)st->fold_den;
  p.coarse_g = (const float*)st->coarse_g;
  p.coarse_on = fu->coarse_on ? 1 : 0;
  p.B = st->batch;
  p.H = st->heads;
  p.keep = st->local_keep;
  p.fine = st->fine_tokens;
  p.group = st->coarse_group;
  p.fine_cap = st->fine_cap;
  p.page_cap = st->page_cap;
  p.sel_cap = st->sel_cap;
  p.pos_hint = -1;
  return p;
}

int check_tokens(const tao_tokens* tok) {
  if (!tok || !tok->q || !tok->k || !tok->v || !tok->raw_q || !tok->raw_k)
    return fail(TAO_E_ARGUMENT, "null token operand");
  if (tok->tokens < 0) return fail(TAO_E_ARGUMENT, "negative token count");
  return TAO_OK;
}

int check_fusion(const tao_fusion* fu) {
  if (!fu || !fu->fusion_a || !fu->fusion_b) return fail(TAO_E_ARGUMENT, "null fusion parameters");
  if (fu->dtype != TAO_BF16 && fu->dtype != TAO_FP32 && fu->dtype != TAO_FP16)
    return fail(TAO_E_ARGUMENT, "fusion dtype must be bf16, fp32 or fp16");
  return TAO_OK;
}

// The association part of `count` seals (fine slots first_slot ..): block
// statistics, C^T into the bank slots, the pending sums in seal order and,
// with page_c, the matrices of the pages these seals complete. The system
// gram + trace / D I is positive definite for finite inputs (its ridge is
// positive), so the solve is not checked here.
hipError_t assoc_seal(const tao_state_dev* st, const tao::TokView& rk, const tao::TokView& v,
                      int64_t new_base, const int64_t* starts, int first_slot, int count,
                      hipStream_t s) {
  const int B = st->batch, H = st->heads, D = st->head_dim;
  const size_t mats = (size_t)st->stats_cap * B * H;
  float* gram = st->stats;
  float* cross = st->stats + mats * D * D;
  for (int done = 0; done < count; done += st->stats_cap) {
    const int n = std::min(st->stats_cap, count - done);
    tao::WriterStatsParams sp{};
    sp.k = rk.p;
    sp.v = v.p;
    sp.k_s[0] = rk.sb; sp.k_s[1] = rk.st; sp.k_s[2] = rk.sh;
    sp.v_s[0] = v.sb; sp.v_s[1] = v.st; sp.v_s[2] = v.sh;
    sp.N = n * B;
    sp.T = st->fine_tokens;
    sp.H = H;
    sp.gram = gram;
    sp.cross = cross;
    sp.starts = starts + done;
    sp.new_base = new_base;
    sp.ring_raw = (const bf16_t*)st->ring_raw;
    sp.ring_v = (const bf16_t*)st->ring_v;
    sp.L = st->local_keep + st->fine_tokens;
    sp.B = B;
    hipError_t e = tao::launch_writer_stats(sp, D, s);
    if (e != hipSuccess) return e;
    tao::AssocSolveParams fp{};
    fp.gram = gram;
    fp.cross = cross;
    fp.count = n * B * H;
    fp.out = (bf16_t*)st->bank_c;
    fp.to_slots = 1;
    fp.B = B;
    fp.H = H;
    fp.cap = st->fine_cap;
    fp.first_slot = first_slot + done;
    fp.group = st->coarse_group;
    e = tao::launch_association_solve(fp, D, s);
    if (e != hipSuccess) return e;
    tao::AssocPendingParams pp{};
    pp.gram = gram;
    pp.cross = cross;
    pp.pending_gram = st->pending_gram;
    pp.pending_cross = st->pending_cross;
    pp.count = n;
    pp.B = B;
    pp.H = H;
    pp.first_slot = first_slot + done;
    pp.group = st->coarse_group;
    pp.reset_pages = st->page_c != nullptr;
    e = tao::launch_assoc_pending(pp, D, s);
    if (e != hipSuccess) return e;
    if (st->page_c) {
      tao::AssocSolveParams pg = fp;
      pg.out = (bf16_t*)st->page_c;
      pg.to_slots = 2;
      pg.cap = st->page_cap;
      pg.fine_first = first_slot + done;
      e = tao::launch_association_solve(pg, D, s);
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// The feature writers' part of `count` seals (fine slots first_slot ..):
// block statistics with the feature mass, C^T into the bank slots
// (association_matrix for the feature-mass writer, structured_matrix over
// the block's 256 tokens for the structured one), z = r(log mass) and the
// run's fp32 mass total for the page descriptors (tao_stream.py:56-65,
// 463-499). page_runs: the mass run (and the statistic sums) restart at each
// page, as with page values and in the full-sequence path; otherwise (the
// streaming index-only state) they sum from the first seal on, as the
// reference's pending_mass / pending_gram / pending_cross /
// pending_square_mass do when no page values are built.
hipError_t feature_seal(const tao_state_dev* st, const tao::TokView& rk, const tao::TokView& v,
                        int64_t new_base, const int64_t* starts, int first_slot, int count,
                        bool page_runs, hipStream_t s) {
  const int B = st->batch, H = st->heads, D = st->head_dim;
  const bool structured = st->fine_writer == TAO_WRITER_STRUCTURED;
  const size_t mats = (size_t)st->stats_cap * B * H;
  float* first = st->stats;                      // gram, or the square mass
  float* cross = st->stats + mats * D * D;
  float* mass = st->stats + 2 * mats * D * D;
  for (int done = 0; done < count; done += st->stats_cap) {
    const int n = std::min(st->stats_cap, count - done);
    tao::WriterStatsParams sp{};
    sp.k = rk.p;
    sp.v = v.p;
    sp.k_s[0] = rk.sb; sp.k_s[1] = rk.st; sp.k_s[2] = rk.sh;
    sp.v_s[0] = v.sb; sp.v_s[1] = v.st; sp.v_s[2] = v.sh;
    sp.N = n * B;
    sp.T = st->fine_tokens;
    sp.H = H;
    sp.mode = structured ? 1 : 0;
    sp.gram = first;
    sp.cross = cross;
    sp.mass = mass;
    sp.starts = starts + done;
    sp.new_base = new_base;
    sp.ring_raw = (const bf16_t*)st->ring_raw;
    sp.ring_v = (const bf16_t*)st->ring_v;
    sp.L = st->local_keep + st->fine_tokens;
    sp.B = B;
    hipError_t e = tao::launch_writer_stats(sp, D, s);
    if (e != hipSuccess) return e;
    if (structured) {
      tao::StructuredParams tp{};
      tp.square = first;
      tp.cross = cross;
      tp.mass = mass;
      tp.count_mats = n * B * H;
      tp.count = (float)st->fine_tokens;
      tp.out = (bf16_t*)st->bank_c;
      tp.to_slots = 1;
      tp.B = B;
      tp.H = H;
      tp.cap = st->fine_cap;
      tp.first_slot = first_slot + done;
      e = tao::launch_structured_matrix(tp, D, s);
    } else {
      tao::AssocSolveParams fp{};
      fp.gram = first;
      fp.cross = cross;
      fp.count = n * B * H;
      fp.out = (bf16_t*)st->bank_c;
      fp.to_slots = 1;
      fp.B = B;
      fp.H = H;
      fp.cap = st->fine_cap;
      fp.first_slot = first_slot + done;
      fp.group = st->coarse_group;
      e = tao::launch_association_solve(fp, D, s);
    }
    if (e != hipSuccess) return e;
    tao::FeatureDescParams dp{};
    dp.mass = mass;
    dp.fine_z = (bf16_t*)st->fine_z;
    dp.fine_mass = st->fine_mass;
    dp.count = n;
    dp.B = B;
    dp.H = H;
    dp.cap = st->fine_cap;
    dp.first_slot = first_slot + done;
    dp.group = st->coarse_group;
    dp.page_runs = page_runs ? 1 : 0;
    e = tao::launch_feature_descriptors(dp, D, s);
    if (e != hipSuccess) return e;
    // (After the descriptors, which read each block's own mass.) The
    // statistics' sums in seal order (tao_stream.py:463-478), restarting at
    // each page with page values; a block that completes a page then holds
    // its page's sums, and the page matrix is the writer's matrix of them
    // (:479-499; structured: over fine_tokens * group tokens). Index-only
    // states that carry the sums keep them running for their snapshots.
    if (st->pending_gram) {
      tao::AssocPendingParams pp{};
      pp.B = B;
      pp.H = H;
      pp.count = n;
      pp.first_slot = first_slot + done;
      pp.group = st->coarse_group;
      pp.reset_pages = page_runs ? 1 : 0;
      if (structured) {
        pp.gram = first;                       // square mass [.., D]
        pp.cross = mass;                       // mass [.., D]
        pp.pending_gram = st->pending_gram;
        pp.pending_cross = st->pending_gram + (size_t)B * H * D;
        e = tao::launch_pending_sums(pp, D, s);
        if (e == hipSuccess) {
          pp.gram = cross;
          pp.cross = nullptr;
          pp.pending_gram = st->pending_cross;
          pp.pending_cross = nullptr;
          e = tao::launch_pending_sums(pp, D * D, s);
        }
        if (e == hipSuccess && st->page_c) {
          tao::StructuredParams tp{};
          tp.square = first;
          tp.cross = cross;
          tp.mass = mass;
          tp.count_mats = n * B * H;
          tp.count = (float)(st->fine_tokens * st->coarse_group);
          tp.out = (bf16_t*)st->page_c;
          tp.to_slots = 2;
          tp.B = B;
          tp.H = H;
          tp.cap = st->page_cap;
          tp.first_slot = first_slot + done;
          tp.group = st->coarse_group;
          e = tao::launch_structured_matrix(tp, D, s);
        }
      } else {
        pp.gram = first;
        pp.cross = cross;
        pp.pending_gram = st->pending_gram;
        pp.pending_cross = st->pending_cross;
        e = tao::launch_assoc_pending(pp, D, s);
        if (e == hipSuccess && st->page_c) {
          tao::AssocSolveParams pg{};
          pg.gram = first;
          pg.cross = cross;
          pg.count = n * B * H;
          pg.out = (bf16_t*)st->page_c;
          pg.to_slots = 2;
          pg.B = B;
          pg.H = H;
          pg.cap = st->page_cap;
          pg.fine_first = first_slot + done;
          pg.group = st->coarse_group;
          e = tao::launch_association_solve(pg, D, s);
        }
      }
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// The regularized writer's share of the backward (association_writer.py:
// 11-32 under autograd): the fines' statistics again, Y = A^{-1} cross and
// W = A^{-1} dC in fp32, S = dG + dG^T, then per block d raw_k's share
// (written to dk_extra) and dv's (added to dv).
struct AssocPages {
  size_t stats, y, w, s;   // workspace offsets
  const float* dpc;        // d page_c [B*H][pages][e][d]
  int pages;
};

// Feature-mass writer (fm non-null): the statistics pass also writes the
// fines' masses, and d mass (from d z of the fines and of the pages' mass
// descriptors) reaches the block adjoint.
struct FeatureMass {
  float* mass; float* dmass;       // [fines * B][H][D]
  const float* dz; const float* dpz;
  int pages;
};

hipError_t assoc_backward(const tao_state_dev* st, const tao_tokens* tok, char* ws,
                          size_t stats_off, size_t y_off, size_t w_off, size_t s_off,
                          size_t dk_off, size_t starts_off, const float* dc, float* dv,
                          int fines, int T, const AssocPages& pg, hipStream_t s,
                          const FeatureMass* fm = nullptr) {
  const int B = st->batch, H = st->heads, D = st->head_dim, ft = st->fine_tokens;
  const int mats = fines * B * H;
  int64_t* starts = (int64_t*)(ws + starts_off);
  hipError_t e = tao::launch_block_starts(starts, fines, ft, s);
  if (e != hipSuccess) return e;
  float* gram = (float*)(ws + stats_off);
  float* cross = gram + (size_t)mats * D * D;
  const tao::TokView rk = view(tok->raw_k, tok->rk_s), vv = view(tok->v, tok->v_s);
  tao::WriterStatsParams sp{};
  sp.k = rk.p;
  sp.v = vv.p;
  sp.k_s[0] = rk.sb; sp.k_s[1] = rk.st; sp.k_s[2] = rk.sh;
  sp.v_s[0] = vv.sb; sp.v_s[1] = vv.st; sp.v_s[2] = vv.sh;
  sp.N = fines * B;
  sp.T = ft;
  sp.H = H;
  sp.gram = gram;
  sp.cross = cross;
  sp.starts = starts;
  sp.new_base = 0;
  sp.ring_raw = (const bf16_t*)st->ring_raw;
  sp.ring_v = (const bf16_t*)st->ring_v;
  sp.L = st->local_keep + st->fine_tokens;
  sp.B = B;
  if (fm) sp.mass = fm->mass;
  e = tao::launch_writer_stats(sp, D, s);
  if (e != hipSuccess) return e;
  tao::AssocSolveParams fp{};
  fp.gram = gram;
  fp.cross = cross;
  fp.count = mats;
  fp.B = B;
  fp.H = H;
  fp.out_f32 = (float*)(ws + y_off);
  e = tao::launch_association_solve(fp, D, s);
  if (e != hipSuccess) return e;
  fp.out_f32 = (float*)(ws + w_off);
  fp.rhs_t = dc;
  fp.rhs_cap = fines;
  e = tao::launch_association_solve(fp, D, s);
  if (e != hipSuccess) return e;
  tao::AssocBwdParams bp{};
  bp.w = (const float*)(ws + w_off);
  bp.y = (const float*)(ws + y_off);
  bp.s = (float*)(ws + s_off);
  bp.raw_k = rk;
  bp.v = vv;
  bp.dk = (float*)(ws + dk_off);
  bp.dv = dv;
  bp.mats = mats;
  bp.B = B;
  bp.H = H;
  bp.T = T;
  bp.ft = ft;
  e = tao::launch_assoc_gram_bwd(bp, D, s);
  if (e != hipSuccess) return e;
  if (pg.pages > 0) {
    // Page g's matrix is the solve of its fines' summed statistics: its
    // adjoints W_g and S_g add to each of its fines' (the sums' gradient).
    const int G = st->coarse_group, pmats = pg.pages * B * H;
    float* pgram = (float*)(ws + pg.stats);
    float* pcross = pgram + (size_t)pmats * D * D;
    e = tao::launch_page_sum(gram, pgram, pg.pages, G, B, H, (int64_t)D * D, s);
    if (e == hipSuccess) e = tao::launch_page_sum(cross, pcross, pg.pages, G, B, H, (int64_t)D * D, s);
    if (e != hipSuccess) return e;
    tao::AssocSolveParams pp{};
    pp.gram = pgram;
    pp.cross = pcross;
    pp.count = pmats;
    pp.B = B;
    pp.H = H;
    pp.out_f32 = (float*)(ws + pg.y);
    e = tao::launch_association_solve(pp, D, s);
    if (e != hipSuccess) return e;
    pp.out_f32 = (float*)(ws + pg.w);
    pp.rhs_t = pg.dpc;
    pp.rhs_cap = pg.pages;
    e = tao::launch_association_solve(pp, D, s);
    if (e != hipSuccess) return e;
    tao::AssocBwdParams gp = bp;
    gp.w = (const float*)(ws + pg.w);
    gp.y = (const float*)(ws + pg.y);
    gp.s = (float*)(ws + pg.s);
    gp.mats = pmats;
    e = tao::launch_assoc_gram_bwd(gp, D, s);
    if (e == hipSuccess)
      e = tao::launch_page_to_fines((float*)(ws + w_off), (float*)(ws + s_off),
                                    (const float*)(ws + pg.w), (const float*)(ws + pg.s), fines, G,
                                    B, H, (int64_t)D * D, s);
    if (e != hipSuccess) return e;
  }
  if (fm) {
    e = tao::launch_mass_grad(fm->dz, fm->dpz, fm->mass, nullptr, fm->dmass, fines, fm->pages,
                              st->coarse_group, B, H, D, s);
    if (e != hipSuccess) return e;
    bp.dmass = fm->dmass;
  }
  return tao::launch_assoc_block_bwd(bp, D, s);
}

// The structured-Gram writer's share of the backward: the fines' statistics
// (square mass, cross, mass) again, the closed form's adjoint per fine and,
// with page values, per completed page (added to its fines'), d mass from
// d z, then per block W = d cross and S = diag(2 d square) through the block
// adjoint (d raw_k's share into dk_off, dv added).
struct StructuredWs {
  size_t stats, mass, w, s, dsq, dms, dmass;        // fines
  size_t pstats, pw, pdsq, pdms;                    // pages
};

hipError_t structured_backward(const tao_state_dev* st, const tao_tokens* tok, char* ws,
                               const StructuredWs& o, size_t dk_off, size_t starts_off,
                               const float* dc, const float* dpc, const float* dz,
                               const float* dpz, float* dv, int fines, int pages, int T,
                               hipStream_t s) {
  const int B = st->batch, H = st->heads, D = st->head_dim, ft = st->fine_tokens;
  const int G = st->coarse_group, mats = fines * B * H;
  int64_t* starts = (int64_t*)(ws + starts_off);
  hipError_t e = tao::launch_block_starts(starts, fines, ft, s);
  if (e != hipSuccess) return e;
  float* square = (float*)(ws + o.stats);
  float* cross = square + (size_t)mats * D * D;
  float* mass = (float*)(ws + o.mass);
  const tao::TokView rk = view(tok->raw_k, tok->rk_s), vv = view(tok->v, tok->v_s);
  tao::WriterStatsParams sp{};
  sp.k = rk.p;
  sp.v = vv.p;
  sp.k_s[0] = rk.sb; sp.k_s[1] = rk.st; sp.k_s[2] = rk.sh;
  sp.v_s[0] = vv.sb; sp.v_s[1] = vv.st; sp.v_s[2] = vv.sh;
  sp.N = fines * B;
  sp.T = ft;
  sp.H = H;
  sp.mode = 1;
  sp.gram = square;
  sp.cross = cross;
  sp.mass = mass;
  sp.starts = starts;
  sp.new_base = 0;
  sp.ring_raw = (const bf16_t*)st->ring_raw;
  sp.ring_v = (const bf16_t*)st->ring_v;
  sp.L = st->local_keep + st->fine_tokens;
  sp.B = B;
  e = tao::launch_writer_stats(sp, D, s);
  if (e != hipSuccess) return e;
  tao::StructuredBwdParams bp{};
  bp.square = square;
  bp.cross = cross;
  bp.mass = mass;
  bp.dct = dc;
  bp.dct_cap = fines;
  bp.B = B;
  bp.H = H;
  bp.count_mats = mats;
  bp.count = (float)ft;
  bp.dsquare = (float*)(ws + o.dsq);
  bp.dcross = (float*)(ws + o.w);
  bp.dmass = (float*)(ws + o.dms);
  e = tao::launch_structured_bwd(bp, D, s);
  if (e != hipSuccess) return e;
  if (pages > 0) {
    // Page p's matrix is the closed form of its fines' summed statistics:
    // its adjoints add to each of its fines'.
    const int pmats = pages * B * H;
    float* psq = (float*)(ws + o.pstats);
    float* pcr = psq + (size_t)pmats * D;
    float* pms = pcr + (size_t)pmats * D * D;
    e = tao::launch_page_sum(square, psq, pages, G, B, H, (int64_t)D, s);
    if (e == hipSuccess) e = tao::launch_page_sum(cross, pcr, pages, G, B, H, (int64_t)D * D, s);
    if (e == hipSuccess) e = tao::launch_page_sum(mass, pms, pages, G, B, H, (int64_t)D, s);
    if (e != hipSuccess) return e;
    tao::StructuredBwdParams pp = bp;
    pp.square = psq;
    pp.cross = pcr;
    pp.mass = pms;
    pp.dct = dpc;
    pp.dct_cap = pages;
    pp.count_mats = pmats;
    pp.count = (float)(ft * G);
    pp.dsquare = (float*)(ws + o.pdsq);
    pp.dcross = (float*)(ws + o.pw);
    pp.dmass = (float*)(ws + o.pdms);
    e = tao::launch_structured_bwd(pp, D, s);
    if (e == hipSuccess)
      e = tao::launch_page_add(bp.dsquare, pp.dsquare, pages, G, B, H, (int64_t)D, s);
    if (e == hipSuccess)
      e = tao::launch_page_add(bp.dcross, pp.dcross, pages, G, B, H, (int64_t)D * D, s);
    if (e == hipSuccess)
      e = tao::launch_page_add(bp.dmass, pp.dmass, pages, G, B, H, (int64_t)D, s);
    if (e != hipSuccess) return e;
  }
  e = tao::launch_square_diag(bp.dsquare, (float*)(ws + o.s), mats, D, s);
  if (e == hipSuccess)
    e = tao::launch_mass_grad(dz, dpz, mass, bp.dmass, (float*)(ws + o.dmass), fines, pages, G, B,
                              H, D, s);
  if (e != hipSuccess) return e;
  tao::AssocBwdParams kb{};
  kb.w = bp.dcross;
  kb.s = (float*)(ws + o.s);
  kb.raw_k = rk;
  kb.v = vv;
  kb.dk = (float*)(ws + dk_off);
  kb.dv = dv;
  kb.mats = mats;
  kb.B = B;
  kb.H = H;
  kb.T = T;
  kb.ft = ft;
  kb.dmass = (const float*)(ws + o.dmass);
  return tao::launch_assoc_block_bwd(kb, D, s);
}

// The captured decode step: one kernel node (the single-launch step with its
// cursor read on the device) instantiated twice. Launches alternate between
// the two executable graphs: re-launching one executable graph while its
// previous launch is still queued makes hipGraphLaunch wait for that launch
// (about 8 us of host time per token on this runtime), two do not.
struct DecodeGraph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec[2] = {nullptr, nullptr};
  hipGraphNode_t step_node = nullptr;    // the graph's only node
  hipKernelNodeParams step_kp{};         // its launch shape (arguments set per launch)
  tao::DecodeParams params{};            // captured arguments; operands replaced per launch
  int32_t selected = 0;
  unsigned next = 0;                     // executable graph of the next launch
};

}  // namespace

namespace tao {

void set_error(const char* msg) { g_error = msg; }

WorkspaceLayout workspace_layout(int batch, int heads, int head_dim, int sel_cap,
                                 int plan_words) {
  auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
  WorkspaceLayout lay;
  const size_t bh = (size_t)batch * heads;
  lay.parts_off = 0;
  const size_t parts = bh * step_floats(head_dim, sel_cap) * sizeof(float);
  lay.count_off = align(parts);
  lay.plan_off =
      align(lay.count_off + step_counters(batch, heads) * kCounterStride * sizeof(unsigned));
  lay.plan_words = plan_words > 0 ? (size_t)plan_words : 0;
  lay.total = align(lay.plan_off + lay.plan_words * sizeof(int64_t));
  return lay;
}

int decode_step_at(const tao_state_dev* st, const tao_tokens* tok, const tao_fusion* fu,
                   int32_t selected, void* out, const int64_t* out_s, void* stream,
                   long long position, float* records, unsigned* counters) {
  if ((records == nullptr) != (counters == nullptr))
    return fail(TAO_E_ARGUMENT, "decode step: records and counters go together");
  int rc = check_state(st, records == nullptr);
  if (!rc) rc = check_tokens(tok);
  if (!rc) rc = check_fusion(fu);
  if (rc) return rc;
  if (tok->tokens != 1) return fail(TAO_E_SHAPE, "decode step takes exactly one token");
  if (!out || !out_s) return fail(TAO_E_ARGUMENT, "null output");
  if (selected < 0 || selected > st->sel_cap) return fail(TAO_E_CAPACITY, "selected count exceeds sel_cap");
  if (fu->coarse_on && !st->coarse_g)
    return fail(TAO_E_ARGUMENT, "coarse_on needs a state with the coarse value branch");
  tao::DecodeParams p = decode_params(st, tok, fu, out, out_s);
  p.pos_hint = position;
  if (records) {
    p.parts = records;
    p.counters = counters;
  }
  return check_hip(tao::launch_decode_step(p, st->head_dim, selected, (hipStream_t)stream),
                   "tao_decode_step");
}

int decode_record(const tao_state_dev* st, const tao_tokens* tok, const tao_fusion* fu,
                  int32_t selected, void* out, const int64_t* out_s, DecodeParams* rec) {
  int rc = check_state(st);
  if (!rc) rc = check_tokens(tok);
  if (!rc) rc = check_fusion(fu);
  if (rc) return rc;
  if (tok->tokens != 1) return fail(TAO_E_SHAPE, "decode step takes exactly one token");
  if (!out || !out_s || !rec) return fail(TAO_E_ARGUMENT, "null output");
  if (selected < 0 || selected > st->sel_cap) return fail(TAO_E_CAPACITY, "selected count exceeds sel_cap");
  if (fu->coarse_on && !st->coarse_g)
    return fail(TAO_E_ARGUMENT, "coarse_on needs a state with the coarse value branch");
  *rec = decode_params(st, tok, fu, out, out_s);
  return TAO_OK;
}

int decode_replay(const DecodeParams& rec, const tao_tokens* tok, int head_dim,
                  int32_t selected, long long position, void* stream) {
  int rc = check_tokens(tok);
  if (rc) return rc;
  if (tok->tokens != 1) return fail(TAO_E_SHAPE, "decode step takes exactly one token");
  DecodeParams p = rec;
  p.q = view(tok->q, tok->q_s);
  p.k = view(tok->k, tok->k_s);
  p.v = view(tok->v, tok->v_s);
  p.rq = view(tok->raw_q, tok->rq_s);
  p.rk = view(tok->raw_k, tok->rk_s);
  p.pos_hint = position;
  return check_hip(tao::launch_decode_step(p, head_dim, selected, (hipStream_t)stream),
                   "decode replay");
}

namespace {

FoldParams fold_params(const tao_state_dev* st, int32_t selected, const TurnGate& gate) {
  FoldParams p{};
  p.bank = (const bf16_t*)st->bank_c;
  p.sw = (const bf16_t*)st->fine_sw;
  p.pw = (const bf16_t*)st->page_w;
  p.sel = st->sel;
  p.fold_g = (float*)st->fold_g;
  p.fold_den = (float*)st->fold_den;
  p.B = st->batch;
  p.H = st->heads;
  p.group = st->coarse_group;
  p.fine_cap = st->fine_cap;
  p.page_cap = st->page_cap;
  p.sel_cap = st->sel_cap;
  p.M = selected;
  p.gate = gate;
  return p;
}

// Checks a single-turn route of the state and fills its parameters.
int route_params(const tao_state_dev* st, const void* raw_q_row, const int64_t* rq_s,
                 int32_t completed, int32_t pending, int32_t coarse, int32_t selected,
                 const TurnGate& gate, RouteParams* out) {
  if (!raw_q_row || !rq_s) return fail(TAO_E_ARGUMENT, "null anchor query");
  const int fines = completed * st->coarse_group + pending;
  if (completed < 0 || pending < 0 || pending >= st->coarse_group || fines <= 0)
    return fail(TAO_E_ARGUMENT, "route needs at least one sealed fine");
  if (fines > st->fine_cap || completed + 1 > st->page_cap)
    return fail(TAO_E_CAPACITY, "route counts exceed the state capacity");
  if (coarse < 0 || coarse > completed || coarse > st->chosen_cap)
    return fail(TAO_E_CAPACITY, "coarse count out of range");
  const int eligible = coarse * st->coarse_group + pending;
  if (selected <= 0 || selected > eligible || selected > st->sel_cap)
    return fail(TAO_E_CAPACITY, "selected count out of range");
  RouteParams p = {};
  p.rq = (const bf16_t*)raw_q_row;
  p.rq_sb = rq_s[0];
  p.rq_st = 0;
  p.rq_sh = rq_s[1];
  p.turns = nullptr;
  p.n_turns = 0;
  p.pw = (const bf16_t*)st->page_w;
  p.sw = (const bf16_t*)st->fine_sw;
  p.sel = st->sel;
  p.chosen = st->chosen;
  p.header = st->header;
  p.B = st->batch;
  p.H = st->heads;
  p.fine_cap = st->fine_cap;
  p.page_cap = st->page_cap;
  p.sel_cap = st->sel_cap;
  p.chosen_cap = st->chosen_cap;
  p.group = st->coarse_group;
  p.completed = completed;
  p.pending = pending;
  p.coarse = coarse;
  p.selected = selected;
  p.gate = gate;
  *out = p;
  return TAO_OK;
}

}  // namespace

int fold_at(const tao_state_dev* st, int32_t selected, const TurnGate& gate, void* stream) {
  int rc = check_state(st);
  if (rc) return rc;
  if (selected < 0 || selected > st->sel_cap) return fail(TAO_E_CAPACITY, "selected count exceeds sel_cap");
  return check_hip(launch_fold(fold_params(st, selected, gate), st->head_dim, (hipStream_t)stream),
                   "tao_fold_route");
}

int route_at(const tao_state_dev* st, const void* raw_q_row, const int64_t* rq_s,
             int32_t completed, int32_t pending, int32_t coarse, int32_t selected,
             const TurnGate& gate, void* stream) {
  int rc = check_state(st);
  if (rc) return rc;
  RouteParams p;
  rc = route_params(st, raw_q_row, rq_s, completed, pending, coarse, selected, gate, &p);
  if (rc) return rc;
  return check_hip(launch_route(p, st->head_dim, (hipStream_t)stream), "tao_route");
}

int refresh_fold_at(const tao_state_dev* st, const void* raw_q_row, const int64_t* rq_s,
                    int32_t completed, int32_t pending, int32_t coarse, int32_t selected,
                    const TurnGate& gate, void* stream) {
  int rc = check_state(st);
  if (rc) return rc;
  RouteParams p;
  rc = route_params(st, raw_q_row, rq_s, completed, pending, coarse, selected, gate, &p);
  if (rc) return rc;
  const FoldParams f = fold_params(st, selected, gate);
  // TAO_REFRESH_FOLD=0 keeps the two launches (the fused kernel computes the
  // same route and fold; the switch exists to compare them).
  const char* env = getenv("TAO_REFRESH_FOLD");
  hipError_t e = hipErrorNotSupported;
  if (!(env && env[0] == '0')) e = launch_refresh_fold(p, f, st->head_dim, (hipStream_t)stream);
  if (e == hipErrorNotSupported) {
    e = launch_route(p, st->head_dim, (hipStream_t)stream);
    if (e == hipSuccess) e = launch_fold(f, st->head_dim, (hipStream_t)stream);
  }
  return check_hip(e, "route refresh");
}

}  // namespace tao

extern "C" {

int tao_abi_version(void) { return TAO_ABI_VERSION; }

const char* tao_last_error(void) { return g_error.c_str(); }

size_t tao_workspace_bytes(int32_t batch, int32_t heads, int32_t head_dim,
                           int32_t sel_cap, int32_t plan_words) {
  return tao::workspace_layout(batch, heads, head_dim, sel_cap, plan_words).total;
}

int tao_workspace_init(const tao_state_dev* st, void* stream) {
  int rc = check_state(st);
  if (rc) return rc;
  return check_hip(hipMemsetAsync(st->workspace, 0, st->workspace_bytes, (hipStream_t)stream),
                   "tao_workspace_init");
}

int tao_decode_step(const tao_state_dev* st, const tao_tokens* tok, const tao_fusion* fu,
                    int32_t selected, void* out, const int64_t* out_s, void* stream) {
  return tao::decode_step_at(st, tok, fu, selected, out, out_s, stream, -1);
}

int tao_fold_route(const tao_state_dev* st, int32_t selected, void* stream) {
  return tao::fold_at(st, selected, tao::TurnGate{}, stream);
}

int tao_page_coarse(const tao_state_dev* st, int32_t first_page, int32_t count, void* stream) {
  int rc = check_state(st);
  if (rc) return rc;
  if (!st->page_c) return fail(TAO_E_ARGUMENT, "state has no coarse value branch");
  if (count < 0 || first_page < 0 || first_page + count > st->page_cap ||
      (int64_t)(first_page + count) * st->coarse_group > st->fine_cap)
    return fail(TAO_E_CAPACITY, "pages exceed the state capacity");
  tao::PageCoarseParams p{};
  p.bank = (const bf16_t*)st->bank_c;
  p.sw = (const bf16_t*)st->fine_sw;
  p.page_c = (bf16_t*)st->page_c;
  p.B = st->batch;
  p.H = st->heads;
  p.fine_cap = st->fine_cap;
  p.page_cap = st->page_cap;
  p.group = st->coarse_group;
  p.first_page = first_page;
  p.count = count;
  return check_hip(tao::launch_page_coarse(p, st->head_dim, (hipStream_t)stream),
                   "tao_page_coarse");
}

int tao_fold_coarse(const tao_state_dev* st, int32_t completed, void* stream) {
  int rc = check_state(st);
  if (rc) return rc;
  if (!st->page_c) return fail(TAO_E_ARGUMENT, "state has no coarse value branch");
  if (completed < 1 || completed > st->page_cap)
    return fail(TAO_E_CAPACITY, "completed pages out of range");
  tao::CoarseFoldParams p{};
  p.page_z = (const bf16_t*)st->page_z;
  p.page_c = (const bf16_t*)st->page_c;
  p.out = st->coarse_g;
  p.out_f32 = 1;
  p.B = st->batch;
  p.H = st->heads;
  p.page_cap = st->page_cap;
  p.n_first = completed;
  p.n_count = 1;
  return check_hip(tao::launch_coarse_fold(p, st->head_dim, (hipStream_t)stream),
                   "tao_fold_coarse");
}

int tao_route(const tao_state_dev* st, const void* raw_q_row, const int64_t* rq_s,
              int32_t completed, int32_t pending, int32_t coarse, int32_t selected,
              void* stream) {
  return tao::route_at(st, raw_q_row, rq_s, completed, pending, coarse, selected,
                       tao::TurnGate{}, stream);
}

int tao_write_fine(const tao_state_dev* st, const tao_tokens* tok, int64_t new_base,
                   const int64_t* start_pos, int32_t first_slot, int32_t count,
                   void* stream) {
  int rc = check_state(st);
  if (!rc) rc = check_tokens(tok);
  if (rc) return rc;
  if (count < 0 || first_slot < 0 || first_slot + count > st->fine_cap)
    return fail(TAO_E_CAPACITY, "fine slots exceed fine_cap");
  if (count && !start_pos) return fail(TAO_E_ARGUMENT, "null block starts");
  tao::WriterParams p{};
  p.rk = view(tok->raw_k, tok->rk_s);
  p.v = view(tok->v, tok->v_s);
  p.ring_raw = (const bf16_t*)st->ring_raw;
  p.ring_v = (const bf16_t*)st->ring_v;
  p.bank = (bf16_t*)st->bank_c;
  p.fine_z = (bf16_t*)st->fine_z;
  p.starts = start_pos;
  p.new_base = new_base;
  p.B = st->batch;
  p.H = st->heads;
  p.L = st->local_keep + st->fine_tokens;
  p.fine_cap = st->fine_cap;
  p.first_slot = first_slot;
  p.count = count;
  p.z_only = assoc_writer(st) ? 1 : 0;
  if (feature_writer(st))
    return check_hip(feature_seal(st, p.rk, p.v, new_base, start_pos, first_slot, count,
                                  st->page_c != nullptr, (hipStream_t)stream),
                     "tao_write_fine");
  hipError_t e = tao::launch_writer(p, st->head_dim, (hipStream_t)stream);
  if (e == hipSuccess && assoc_writer(st) && count > 0)
    e = assoc_seal(st, p.rk, p.v, new_base, start_pos, first_slot, count, (hipStream_t)stream);
  return check_hip(e, "tao_write_fine");
}

int tao_seal_epilogue(const tao_state_dev* st, int32_t slot, int32_t pages, int32_t recompute,
                      void* stream) {
  int rc = check_state(st);
  if (rc) return rc;
  if (slot < 0 || slot >= st->fine_cap) return fail(TAO_E_CAPACITY, "slot exceeds fine_cap");
  if (pages != slot / st->coarse_group + 1 || pages > st->page_cap)
    return fail(TAO_E_ARGUMENT, "pages must be slot / coarse_group + 1 and fit page_cap");
  tao::EpilogueParams p{};
  p.fine_z = (const bf16_t*)st->fine_z;
  p.fine_sw = (bf16_t*)st->fine_sw;
  p.page_z = (bf16_t*)st->page_z;
  p.page_w = (bf16_t*)st->page_w;
  p.fine_mass = st->fine_mass;
  p.B = st->batch;
  p.H = st->heads;
  p.fine_cap = st->fine_cap;
  p.page_cap = st->page_cap;
  p.group = st->coarse_group;
  p.slot = slot;
  p.pages = pages;
  p.recompute = recompute ? 1 : 0;
  return check_hip(tao::launch_seal_epilogue(p, st->head_dim, (hipStream_t)stream),
                   "tao_seal_epilogue");
}

int tao_local_attention(const tao_state_dev* st, const tao_tokens* tok, int64_t qpos0,
                        int64_t kpos0, const int64_t* tiles, int32_t n_tiles, void* local,
                        void* stream) {
  int rc = check_state(st);
  if (!rc) rc = check_tokens(tok);
  if (rc) return rc;
  if (!local) return fail(TAO_E_ARGUMENT, "null local output");
  if (n_tiles < 0 || (n_tiles && !tiles)) return fail(TAO_E_ARGUMENT, "bad tile list");
  tao::AttnParams p{};
  p.q = view(tok->q, tok->q_s);
  p.k = view(tok->k, tok->k_s);
  p.v = view(tok->v, tok->v_s);
  p.ring_k = (const bf16_t*)st->ring_k;
  p.ring_v = (const bf16_t*)st->ring_v;
  p.out = (bf16_t*)local;
  p.tiles = tiles;
  p.qpos0 = qpos0;
  p.kpos0 = kpos0;
  p.B = st->batch;
  p.H = st->heads;
  p.L = st->local_keep + st->fine_tokens;
  p.T = tok->tokens;
  p.n_tiles = n_tiles;
  return check_hip(tao::launch_local_attention(p, st->head_dim, (hipStream_t)stream),
                   "tao_local_attention");
}

int tao_prompt_attention(const tao_stream_cfg* cfg, int32_t batch, int32_t heads,
                         int32_t head_dim, const tao_tokens* tok, int64_t pos0,
                         void* tiles_dev, int64_t tiles_cap, void* local, void* stream) {
  int rc = check_tokens(tok);
  if (rc) return rc;
  if (!cfg || batch < 1 || heads < 1 || (head_dim != 64 && head_dim != 128) ||
      cfg->local_keep < 0 || cfg->fine_tokens < 1)
    return fail(TAO_E_ARGUMENT, "prompt attention: bad geometry");
  if (!local || !tiles_dev || pos0 < 0) return fail(TAO_E_ARGUMENT, "prompt attention: null tiles or output");
  const int64_t L = tao::sched::serve_limit(*cfg), T = tok->tokens;
  std::vector<int64_t> tiles;
  bool inside = true;
  tao::sched::attention_tiles(*cfg, pos0, T, [&](int64_t row, int64_t n, int64_t key_start) {
    inside = inside && key_start >= pos0 && key_start <= pos0 + row && pos0 + row + n - key_start <= L;
    tiles.insert(tiles.end(), {row, n, key_start});
  });
  if (!inside) return fail(TAO_E_ARGUMENT, "prompt attention: the window reaches before the call");
  const int64_t n_tiles = (int64_t)tiles.size() / 3;
  if (3 * n_tiles > tiles_cap) return fail(TAO_E_CAPACITY, "prompt attention: tiles_cap too small");
  if (n_tiles == 0) return TAO_OK;
  const hipStream_t s = (hipStream_t)stream;
  hipError_t e = hipMemcpyAsync(tiles_dev, tiles.data(), tiles.size() * sizeof(int64_t),
                                hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return check_hip(e, "tao_prompt_attention");
  tao::AttnParams ap{};
  ap.q = view(tok->q, tok->q_s);
  ap.k = view(tok->k, tok->k_s);
  ap.v = view(tok->v, tok->v_s);
  ap.ring_k = nullptr;   // every key is one of the call's (checked above)
  ap.ring_v = nullptr;
  ap.out = (bf16_t*)local;
  ap.tiles = (const int64_t*)tiles_dev;
  ap.qpos0 = pos0;
  ap.kpos0 = pos0;
  ap.B = batch;
  ap.H = heads;
  ap.L = (int)L;
  ap.T = (int)T;
  ap.n_tiles = (int)n_tiles;
  ap.lse = nullptr;
  return check_hip(tao::launch_local_attention(ap, head_dim, s), "tao_prompt_attention");
}

int tao_prefill(const tao_state_dev* st, const tao_tokens* tok, const tao_fusion* fu,
                const int64_t* plan, int64_t plan_len, const tao_prefill_pools* pools,
                void* local, void* out, const int64_t* out_s, void* stream) {
  int rc = check_state(st);
  if (!rc) rc = check_tokens(tok);
  if (!rc) rc = check_fusion(fu);
  if (rc) return rc;
  if (!plan || plan_len < TAO_PLAN_HEADER || !local || !out || !out_s)
    return fail(TAO_E_ARGUMENT, "null plan, local or output");
  if ((size_t)plan_len > plan_capacity(st))
    return fail(TAO_E_WORKSPACE, "prefill plan larger than the workspace plan region");
  const hipStream_t s = (hipStream_t)stream;
  const int T = tok->tokens;
  const int L = st->local_keep + st->fine_tokens;
  const int64_t pos0 = plan[TAO_PLAN_POS0];
  if (pos0 < 0) return fail(TAO_E_ARGUMENT, "negative position");
  const int64_t window0 = pos0 - [&] {
    if (pos0 < L) return (int64_t)pos0;
    return (int64_t)st->local_keep + (pos0 - L) % st->fine_tokens;
  }();
  // ---- section offsets
  const int64_t n_attn = plan[TAO_PLAN_ATTN_TILES], n_write = plan[TAO_PLAN_WRITES];
  const int64_t n_turns = plan[TAO_PLAN_TURNS], n_read = plan[TAO_PLAN_READ_TILES];
  if (n_attn < 0 || n_write < 0 || n_turns < 0 || n_read < 0)
    return fail(TAO_E_ARGUMENT, "negative plan section");
  const int64_t off_attn = TAO_PLAN_HEADER, off_write = off_attn + 3 * n_attn;
  const int64_t off_turns = off_write + n_write, off_read = off_turns + 8 * n_turns;
  if (off_read + 8 * n_read != plan_len) return fail(TAO_E_ARGUMENT, "plan length mismatch");
  const int64_t query_mode = plan[TAO_PLAN_QUERY_ROUTES];
  if (query_mode != 0 && query_mode != 1) return fail(TAO_E_ARGUMENT, "invalid route mode");
  const bool query_routes = query_mode == 1;
  if (query_routes && n_turns) return fail(TAO_E_ARGUMENT, "per-query routes take no turns");
  const int BH = st->batch * st->heads;
  // ---- validate attention tiles
  for (int64_t i = 0; i < n_attn; ++i) {
    const int64_t* t = plan + off_attn + 3 * i;
    if (t[0] < 0 || t[1] < 1 || t[1] > 256 || t[0] + t[1] > T)
      return fail(TAO_E_ARGUMENT, "attention tile outside the call's tokens");
    if (t[2] < window0 || t[2] > pos0 + t[0] || pos0 + t[0] + t[1] - t[2] > L)
      return fail(TAO_E_ARGUMENT, "attention tile window outside the local ring");
  }
  // ---- writer blocks
  const int64_t first_slot = plan[TAO_PLAN_FIRST_SLOT];
  for (int64_t i = 0; i < n_write; ++i) {
    const int64_t b0 = plan[off_write + i];
    if (b0 < window0 || b0 + st->fine_tokens > pos0 + T)
      return fail(TAO_E_ARGUMENT, "writer block outside the ring and the call's tokens");
  }
  if (n_write && (first_slot < 0 || first_slot + n_write > st->fine_cap))
    return fail(TAO_E_CAPACITY, "written fines exceed fine_cap");
  // ---- pages and epochs
  const int64_t first_page = plan[TAO_PLAN_FIRST_PAGE], n_pages = plan[TAO_PLAN_PAGES];
  const int64_t first_epoch = plan[TAO_PLAN_FIRST_EPOCH], n_epochs = plan[TAO_PLAN_EPOCHS];
  const int G = st->coarse_group;
  if (n_pages < 0 || (n_pages && (first_page < 0 || first_page + n_pages > st->page_cap ||
                                  (first_page + n_pages) * G > st->fine_cap)))
    return fail(TAO_E_CAPACITY, "completed pages exceed the state capacity");
  if (n_epochs < 0) return fail(TAO_E_ARGUMENT, "negative epoch count");
  const bool need_pools = n_epochs > 0 || n_turns > 0;
  if (need_pools) {
    if (!pools || !pools->pw_pool || !pools->psw_pool || (!query_routes && !pools->sel_pool))
      return fail(TAO_E_ARGUMENT, "prefill with history needs epoch pools");
    if (query_routes && (!pools->qsel || pools->qsel_words < 1 || pools->qsel_words > 512))
      return fail(TAO_E_ARGUMENT, "per-query routes need the qsel bitmask pool");
    const int64_t last = first_epoch + n_epochs - 1;
    if (first_epoch < 1 || n_epochs > pools->epochs || last > st->fine_cap ||
        last / G + 1 > pools->pool_pcap || last / G + 1 > st->page_cap)
      return fail(TAO_E_CAPACITY, "epoch range exceeds the pools or the state");
  }
  // ---- turns
  for (int64_t i = 0; i < n_turns; ++i) {
    const int64_t* t = plan + off_turns + 8 * i;
    const int64_t epoch = first_epoch + t[1];
    const int64_t eligible = t[4] * G + t[3];
    if (t[0] < 0 || t[0] >= T || t[1] < 0 || t[1] >= n_epochs ||
        t[2] * G + t[3] != epoch || t[3] < 0 || t[3] >= G || t[4] < 0 || t[4] > t[2] ||
        t[5] < 1 || t[5] > eligible || t[5] > st->sel_cap || t[6] < 1 ||
        t[6] >= pools->sel_slots || (t[7] != 0 && t[7] != 1) || t[2] > 2048 ||
        eligible > 2048 || t[4] > st->chosen_cap)
      return fail(TAO_E_ARGUMENT, "invalid route turn in the plan");
  }
  // ---- read tiles
  if (n_read > 0 && need_pools && st->fine_cap > 16384)
    return fail(TAO_E_CAPACITY, "prefill reads index at most 16384 fines per state");
  const bool coarse_values = st->page_c != nullptr;
  const int external_values = pools && pools->external_values ? 1 : 0;
  const int64_t c_first = pools ? pools->coarse_first : 0;
  const int64_t c_count = pools ? pools->coarse_count : 0;
  bool coarse_reads = false;
  for (int64_t i = 0; i < n_read; ++i) {
    const int64_t* t = plan + off_read + 8 * i;
    if (t[0] < 0 || t[1] < 1 || t[1] > 32 || t[0] + t[1] > T || (t[6] != 0 && t[6] != 1))
      return fail(TAO_E_ARGUMENT, "invalid read tile in the plan");
    if (t[6]) {
      const int64_t epoch = first_epoch + t[4];
      if (!pools || t[4] < 0 || t[4] >= n_epochs || t[5] != (epoch / G) * G || t[7] != epoch / G)
        return fail(TAO_E_ARGUMENT, "invalid history read tile in the plan");
      if (query_routes) {
        // t[2] = coarse pages, t[3] = selected of the tile's epoch
        const int64_t K = epoch / G, eligible = t[2] * G + epoch % G;
        if (t[2] < 0 || t[2] > K || t[3] < 1 || t[3] > eligible ||
            eligible > tao::kQueryRouteMaxKeys || K > tao::kQueryRouteMaxKeys || epoch > 1024 ||
            (epoch + 31) / 32 > pools->qsel_words)
          return fail(TAO_E_ARGUMENT, "invalid per-query read tile in the plan");
      } else if (t[2] < 0 || t[2] >= pools->sel_slots || t[3] < 1 || t[3] > 128 ||
                 t[3] > st->sel_cap) {
        return fail(TAO_E_ARGUMENT, "invalid history read tile in the plan");
      }
      if (coarse_values && t[7] >= 1) {
        if (!pools->coarse_pool || t[7] < c_first || t[7] >= c_first + c_count)
          return fail(TAO_E_ARGUMENT, "coarse read outside the coarse pool");
        coarse_reads = true;
      }
    } else if (t[7] != 0) {
      return fail(TAO_E_ARGUMENT, "invalid read tile in the plan");
    }
  }
  if (coarse_reads && (c_first < 1 || c_first + c_count - 1 > st->page_cap ||
                       c_first + c_count - 1 > first_page + n_pages))
    return fail(TAO_E_CAPACITY, "coarse pool range exceeds the completed pages");
  // ---- ring append
  const int64_t ring_first = plan[TAO_PLAN_RING_FIRST], ring_count = plan[TAO_PLAN_RING_COUNT];
  if (ring_first < 0 || ring_count < 0 || ring_first + ring_count > T || ring_count > L ||
      plan[TAO_PLAN_RING_POS] != pos0 + ring_first)
    return fail(TAO_E_ARGUMENT, "invalid ring append in the plan");

  int64_t* dplan = plan_of(st);
  hipError_t e = hipMemcpyAsync(dplan, plan, (size_t)plan_len * sizeof(int64_t),
                                hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return check_hip(e, "tao_prefill plan upload");
  if (!query_routes && need_pools && pools->sel_slots > 0) {
    e = hipMemcpyAsync(pools->sel_pool, st->sel, (size_t)BH * st->sel_cap * sizeof(int32_t),
                       hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return check_hip(e, "tao_prefill route carry");
  }
  const int D = st->head_dim;
  // local attention
  tao::AttnParams ap{};
  ap.q = view(tok->q, tok->q_s);
  ap.k = view(tok->k, tok->k_s);
  ap.v = view(tok->v, tok->v_s);
  ap.ring_k = (const bf16_t*)st->ring_k;
  ap.ring_v = (const bf16_t*)st->ring_v;
  ap.out = (bf16_t*)local;
  ap.tiles = dplan + off_attn;
  ap.qpos0 = pos0;
  ap.kpos0 = pos0;
  ap.B = st->batch;
  ap.H = st->heads;
  ap.L = L;
  ap.T = T;
  ap.n_tiles = (int)n_attn;
  ap.lse = pools ? pools->local_lse : nullptr;
  e = tao::launch_local_attention(ap, D, s);
  if (e != hipSuccess) return check_hip(e, "tao_prefill attention");
  // writer
  tao::WriterParams wp{};
  wp.rk = view(tok->raw_k, tok->rk_s);
  wp.v = view(tok->v, tok->v_s);
  wp.ring_raw = (const bf16_t*)st->ring_raw;
  wp.ring_v = (const bf16_t*)st->ring_v;
  wp.bank = (bf16_t*)st->bank_c;
  wp.fine_z = (bf16_t*)st->fine_z;
  wp.starts = dplan + off_write;
  wp.new_base = pos0;
  wp.B = st->batch;
  wp.H = st->heads;
  wp.L = L;
  wp.fine_cap = st->fine_cap;
  wp.first_slot = (int)first_slot;
  wp.count = (int)n_write;
  wp.z_only = external_values || assoc_writer(st);
  if (feature_writer(st)) {
    if (external_values) return fail(TAO_E_ARGUMENT, "external values with a feature writer");
    e = feature_seal(st, wp.rk, wp.v, pos0, wp.starts, (int)first_slot, (int)n_write,
                     st->page_c != nullptr || query_routes, s);
  } else {
    e = tao::launch_writer(wp, D, s);
  }
  if (e != hipSuccess) return check_hip(e, "tao_prefill writer");
  if (assoc_writer(st) && n_write > 0) {
    e = assoc_seal(st, wp.rk, wp.v, pos0, wp.starts, (int)first_slot, (int)n_write, s);
    if (e != hipSuccess) return check_hip(e, "tao_prefill association writer");
  }
  // pages
  tao::PagesParams pp{};
  pp.fine_z = (const bf16_t*)st->fine_z;
  pp.fine_sw = (bf16_t*)st->fine_sw;
  pp.page_z = (bf16_t*)st->page_z;
  pp.fine_mass = st->fine_mass;
  pp.B = st->batch;
  pp.H = st->heads;
  pp.fine_cap = st->fine_cap;
  pp.page_cap = st->page_cap;
  pp.group = G;
  pp.first_page = (int)first_page;
  pp.count = (int)n_pages;
  e = tao::launch_pages(pp, D, s);
  if (e != hipSuccess) return check_hip(e, "tao_prefill pages");
  if (coarse_values && !external_values && !assoc_writer(st) && !feature_writer(st)) {
    tao::PageCoarseParams cp{};
    cp.bank = (const bf16_t*)st->bank_c;
    cp.sw = (const bf16_t*)st->fine_sw;
    cp.page_c = (bf16_t*)st->page_c;
    cp.B = st->batch;
    cp.H = st->heads;
    cp.fine_cap = st->fine_cap;
    cp.page_cap = st->page_cap;
    cp.group = G;
    cp.first_page = (int)first_page;
    cp.count = (int)n_pages;
    e = tao::launch_page_coarse(cp, D, s);
    if (e != hipSuccess) return check_hip(e, "tao_prefill page values");
  }
  if (coarse_reads && !feature_writer(st)) {   // feature writers mix pages per query
    tao::CoarseFoldParams cf{};
    cf.page_z = (const bf16_t*)st->page_z;
    cf.page_c = (const bf16_t*)st->page_c;
    cf.out = pools->coarse_pool;
    cf.out_f32 = 0;
    cf.B = st->batch;
    cf.H = st->heads;
    cf.page_cap = st->page_cap;
    cf.n_first = (int)c_first;
    cf.n_count = (int)c_count;
    e = tao::launch_coarse_fold(cf, D, s);
    if (e != hipSuccess) return check_hip(e, "tao_prefill coarse fold");
  }
  if (need_pools) {
    tao::EpochParams ep{};
    ep.fine_z = (const bf16_t*)st->fine_z;
    ep.fine_sw = (bf16_t*)st->fine_sw;
    ep.page_z = (bf16_t*)st->page_z;
    ep.page_w = (bf16_t*)st->page_w;
    ep.fine_mass = st->fine_mass;
    ep.pw_pool = (bf16_t*)pools->pw_pool;
    ep.psw_pool = (bf16_t*)pools->psw_pool;
    ep.pool_pcap = pools->pool_pcap;
    ep.B = st->batch;
    ep.H = st->heads;
    ep.fine_cap = st->fine_cap;
    ep.page_cap = st->page_cap;
    ep.group = G;
    ep.first_epoch = (int)first_epoch;
    ep.count = (int)n_epochs;
    e = tao::launch_epochs(ep, D, s);
    if (e != hipSuccess) return check_hip(e, "tao_prefill epochs");
  }
  if (n_turns) {
    tao::RouteParams rp = {};
    rp.rq = (const bf16_t*)tok->raw_q;
    rp.rq_sb = tok->rq_s[0];
    rp.rq_st = tok->rq_s[1];
    rp.rq_sh = tok->rq_s[2];
    rp.pw = (const bf16_t*)st->page_w;
    rp.sw = (const bf16_t*)st->fine_sw;
    rp.pw_pool = (const bf16_t*)pools->pw_pool;
    rp.psw_pool = (const bf16_t*)pools->psw_pool;
    rp.pool_pcap = pools->pool_pcap;
    rp.sel = st->sel;
    rp.chosen = st->chosen;
    rp.header = st->header;
    rp.sel_pool = pools->sel_pool;
    rp.turns = dplan + off_turns;
    rp.n_turns = (int)n_turns;
    rp.B = st->batch;
    rp.H = st->heads;
    rp.fine_cap = st->fine_cap;
    rp.page_cap = st->page_cap;
    rp.sel_cap = st->sel_cap;
    rp.chosen_cap = st->chosen_cap;
    rp.group = G;
    rp.max_epoch = (int)(first_epoch + n_epochs - 1);
    e = tao::launch_route(rp, D, s);
    if (e != hipSuccess) return check_hip(e, "tao_prefill routes");
  }
  if (query_routes && need_pools && n_read) {
    tao::QueryRouteParams qp{};
    qp.rq = (const bf16_t*)tok->raw_q;
    qp.rq_sb = tok->rq_s[0];
    qp.rq_st = tok->rq_s[1];
    qp.rq_sh = tok->rq_s[2];
    qp.sw = (const bf16_t*)st->fine_sw;
    qp.pw_pool = (const bf16_t*)pools->pw_pool;
    qp.psw_pool = (const bf16_t*)pools->psw_pool;
    qp.pool_pcap = pools->pool_pcap;
    qp.tiles = dplan + off_read;
    qp.n_tiles = (int)n_read;
    qp.qsel = pools->qsel;
    qp.qsel_words = pools->qsel_words;
    qp.first_epoch = (int)first_epoch;
    qp.max_epoch = (int)(first_epoch + n_epochs - 1);
    qp.B = st->batch;
    qp.H = st->heads;
    qp.T = T;
    qp.group = G;
    qp.fine_cap = st->fine_cap;
    e = tao::launch_route_queries(qp, D, s);
    if (e != hipSuccess) return check_hip(e, "tao_prefill per-query routes");
  }
  tao::ReadTilesParams rt{};
  rt.rq = view(tok->raw_q, tok->rq_s);
  rt.bank = (const bf16_t*)st->bank_c;
  rt.sw = (const bf16_t*)st->fine_sw;
  rt.pw_pool = need_pools ? (const bf16_t*)pools->pw_pool : nullptr;
  rt.psw_pool = need_pools ? (const bf16_t*)pools->psw_pool : nullptr;
  rt.pool_pcap = need_pools ? pools->pool_pcap : 0;
  rt.sel_pool = need_pools ? pools->sel_pool : nullptr;
  rt.local = (const bf16_t*)local;
  rt.fa = fu->fusion_a;
  rt.fb = fu->fusion_b;
  rt.f_dtype = fu->dtype;
  for (int i = 0; i < 3; ++i) { rt.fa_s[i] = fu->a_s[i]; rt.fb_s[i] = fu->b_s[i]; }
  rt.gain = fu->gain;
  rt.out = (bf16_t*)out;
  rt.out_sb = out_s[0];
  rt.out_st = out_s[1];
  rt.out_sh = out_s[2];
  rt.tiles = dplan + off_read;
  rt.n_tiles = (int)n_read;
  rt.B = st->batch;
  rt.H = st->heads;
  rt.T = T;
  rt.group = G;
  rt.fine_cap = st->fine_cap;
  rt.sel_cap = st->sel_cap;
  rt.coarse_pool = coarse_reads ? (const bf16_t*)pools->coarse_pool : nullptr;
  rt.coarse_first = coarse_reads ? (int)c_first : 0;
  rt.qsel = query_routes && need_pools ? pools->qsel : nullptr;
  rt.qsel_words = query_routes && need_pools ? pools->qsel_words : 0;
  rt.first_epoch = (int)first_epoch;
  rt.save_coarse = pools ? (bf16_t*)pools->coarse_out : nullptr;
  rt.save_fine = pools ? (bf16_t*)pools->fine_out : nullptr;
  rt.save_den = pools ? pools->den_out : nullptr;
  rt.fine_z = feature_writer(st) ? (const bf16_t*)st->fine_z : nullptr;
  if (feature_writer(st) && coarse_reads) {
    rt.coarse_pool = nullptr;
    rt.page_z = (const bf16_t*)st->page_z;
    rt.page_c = (const bf16_t*)st->page_c;
    rt.page_cap = st->page_cap;
  }
  if (feature_writer(st) && rt.save_fine && !query_routes)
    return fail(TAO_E_ARGUMENT, "a feature writer's turn-route read keeps no saves");
  e = tao::launch_read_tiles(rt, D, s);
  if (e != hipSuccess) return check_hip(e, "tao_prefill read");
  tao::AppendParams app{};
  app.k = view(tok->k, tok->k_s);
  app.v = view(tok->v, tok->v_s);
  app.rk = view(tok->raw_k, tok->rk_s);
  app.ring_k = (bf16_t*)st->ring_k;
  app.ring_v = (bf16_t*)st->ring_v;
  app.ring_raw = (bf16_t*)st->ring_raw;
  app.B = st->batch;
  app.H = st->heads;
  app.D = D;
  app.L = L;
  app.first = (int)ring_first;
  app.count = (int)ring_count;
  app.pos = pos0 + ring_first;
  return check_hip(tao::launch_ring_append(app, s), "tao_prefill ring");
}

int tao_ring_append(const tao_state_dev* st, const tao_tokens* tok, int32_t first,
                    int32_t count, int64_t pos, void* stream) {
  int rc = check_state(st);
  if (!rc) rc = check_tokens(tok);
  if (rc) return rc;
  const int L = st->local_keep + st->fine_tokens;
  if (first < 0 || count < 0 || first + count > tok->tokens || count > L)
    return fail(TAO_E_ARGUMENT, "ring append range out of bounds");
  tao::AppendParams p{};
  p.k = view(tok->k, tok->k_s);
  p.v = view(tok->v, tok->v_s);
  p.rk = view(tok->raw_k, tok->rk_s);
  p.ring_k = (bf16_t*)st->ring_k;
  p.ring_v = (bf16_t*)st->ring_v;
  p.ring_raw = (bf16_t*)st->ring_raw;
  p.B = st->batch;
  p.H = st->heads;
  p.D = st->head_dim;
  p.L = L;
  p.first = first;
  p.count = count;
  p.pos = pos;
  return check_hip(tao::launch_ring_append(p, (hipStream_t)stream), "tao_ring_append");
}

int tao_graph_create(const tao_state_dev* st, const tao_fusion* fu, int32_t selected,
                     void* staging, void* out_stage, void* stream, void** graph_out) {
  int rc = check_state(st);
  if (!rc) rc = check_fusion(fu);
  if (rc) return rc;
  (void)staging;   // unused: the step reads the operands where the caller holds them
  if (!out_stage || !graph_out) return fail(TAO_E_ARGUMENT, "null graph buffers");
  if (st->page_c || fu->coarse_on)
    return fail(TAO_E_ARGUMENT, "the decode hipGraph implements the index-only coarse preset");
  if (selected < 0 || selected > st->sel_cap) return fail(TAO_E_CAPACITY, "selected out of range");
  const int D = st->head_dim;
  // Captured with out_stage as every operand (a [B,1,H,D] buffer, so the
  // captured arguments stay in bounds); each launch replaces them before the
  // graph runs.
  tao_tokens tok{};
  tok.q = tok.k = tok.v = tok.raw_q = tok.raw_k = out_stage;
  const int64_t s[3] = {(int64_t)st->heads * D, 0, (int64_t)D};
  for (int i = 0; i < 3; ++i) {
    tok.q_s[i] = s[i]; tok.k_s[i] = s[i]; tok.v_s[i] = s[i]; tok.rq_s[i] = s[i]; tok.rk_s[i] = s[i];
  }
  tok.tokens = 1;
  DecodeGraph* g = new DecodeGraph();
  g->params = decode_params(st, &tok, fu, out_stage, s);
  g->selected = selected;
  hipStream_t cs = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&cs, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
  if (e == hipSuccess) {
    const hipError_t le = tao::launch_decode_step(g->params, D, selected, cs);
    e = hipStreamEndCapture(cs, &g->graph);
    if (e == hipSuccess) e = le;
  }
  if (e == hipSuccess) {
    size_t nodes = 0;
    e = hipGraphGetNodes(g->graph, nullptr, &nodes);
    if (e == hipSuccess && nodes != 1) e = hipErrorInvalidValue;
    if (e == hipSuccess) e = hipGraphGetNodes(g->graph, &g->step_node, &nodes);
    hipGraphNodeType type = hipGraphNodeTypeEmpty;
    if (e == hipSuccess) e = hipGraphNodeGetType(g->step_node, &type);
    if (e == hipSuccess && type != hipGraphNodeTypeKernel) e = hipErrorInvalidValue;
    if (e == hipSuccess) e = hipGraphKernelNodeGetParams(g->step_node, &g->step_kp);
  }
  for (int i = 0; i < 2 && e == hipSuccess; ++i)
    e = hipGraphInstantiate(&g->exec[i], g->graph, nullptr, nullptr, 0);
  if (cs) (void)hipStreamDestroy(cs);
  if (e != hipSuccess) {
    for (hipGraphExec_t x : g->exec)
      if (x) (void)hipGraphExecDestroy(x);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
    return check_hip(e, "tao_graph_create");
  }
  (void)stream;
  *graph_out = g;
  return TAO_OK;
}

int tao_graph_launch(void* graph, const tao_tokens* tok, void* stream) {
  if (!graph) return fail(TAO_E_ARGUMENT, "null graph");
  int rc = check_tokens(tok);
  if (rc) return rc;
  if (tok->tokens != 1) return fail(TAO_E_SHAPE, "decode step takes exactly one token");
  DecodeGraph* g = (DecodeGraph*)graph;
  tao::DecodeParams p = g->params;
  p.q = view(tok->q, tok->q_s);
  p.k = view(tok->k, tok->k_s);
  p.v = view(tok->v, tok->v_s);
  p.rq = view(tok->raw_q, tok->rq_s);
  p.rk = view(tok->raw_k, tok->rk_s);
  // Point the step at this call's operands; launches already queued keep
  // the arguments they were launched with.
  int32_t selected = g->selected;
  void* args[2] = {&p, &selected};
  hipKernelNodeParams kp = g->step_kp;
  kp.kernelParams = args;
  kp.extra = nullptr;
  hipGraphExec_t x = g->exec[g->next];
  hipError_t e = hipGraphExecKernelNodeSetParams(x, g->step_node, &kp);
  if (e == hipSuccess) e = hipGraphLaunch(x, (hipStream_t)stream);
  if (e == hipSuccess) g->next ^= 1u;
  return check_hip(e, "tao_graph_launch");
}

int tao_graph_destroy(void* graph) {
  if (!graph) return TAO_OK;
  DecodeGraph* g = (DecodeGraph*)graph;
  hipError_t e = hipSuccess;
  for (hipGraphExec_t x : g->exec)
    if (x) {
      const hipError_t d = hipGraphExecDestroy(x);
      if (e == hipSuccess) e = d;
    }
  if (g->graph) (void)hipGraphDestroy(g->graph);
  delete g;
  return check_hip(e, "tao_graph_destroy");
}

int tao_step_stamps(void* buf, int64_t frames, int64_t frame_words) {
  if (tao::step_stamps_set(buf, frames, frame_words))
    return fail(TAO_E_ARGUMENT, "tao_step_stamps: frames must be positive and frames of at "
                                "least 8 words");
  return TAO_OK;
}

int64_t tao_step_stamps_count(void) { return tao::step_stamps_count(); }

}  // extern "C"

// ---------------------------------------------------------------------------
// Full-sequence backward (train_bwd.hip).
namespace {

struct TrainBwdLayout {
  size_t dlocal, h, delta, dden, dcoarse, dnum, drq, dh, dvf;   // per-token arrays
  size_t dpw, dsw_tile, dgc, dc, dsw, dpz, dz, dalpha;          // memory branch, d alpha
  size_t dalpha_parts;                                          // per fusion workgroup
  // regularized writer: statistics, solutions Y and W, S, d raw_k share, starts;
  // with page values, the pages' statistic sums, Y, W, S and d page_c
  size_t stats, sol_y, sol_w, sgram, dk_extra, starts;
  size_t pstats, psol_y, psol_w, psgram, dpc;
  // feature writers: masses, d mass, structured adjoints, d z of the fines'
  // and pages' descriptors, the mixture weights and d masses per query rank
  size_t fmass, fdmass, fdsq, fdms, fdz, fdpz, wv, dmv, pdsq, pdms;
  size_t zero_begin, zero_end;                                  // accumulators to clear
  size_t total;
  int n_tiles, v_max;
};

TrainBwdLayout train_bwd_layout(const tao_state_dev* st, int64_t tokens, int fines,
                                const tao_prefill_pools* pools) {
  TrainBwdLayout l{};
  const size_t B = st->batch, H = st->heads, D = st->head_dim, T = (size_t)tokens;
  const size_t rows = B * T * H, BH = B * H;
  const size_t pcap = pools ? (size_t)pools->pool_pcap : 0;
  const size_t cc = pools ? (size_t)pools->coarse_count : 0;
  l.n_tiles = (int)((tokens + st->fine_tokens - 1) / st->fine_tokens);
  l.v_max = fines;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) & ~(size_t)255;
    return o;
  };
  l.dlocal = take(rows * D * 2);
  l.h = take(rows * D * 2);
  l.delta = take(rows * 4);
  l.dden = take(rows * 4);
  l.dcoarse = take(rows * D * 4);
  l.dnum = take(rows * D * 4);
  l.drq = take(rows * D * 4);
  l.dh = take(rows * D * 4);
  l.dvf = take(rows * D * 4);
  l.zero_begin = off;
  l.dgc = take(cc * BH * D * D * 4);
  l.dc = take(BH * (size_t)fines * D * D * 4);
  l.dpw = take((size_t)l.n_tiles * BH * pcap * D * 4);
  l.dsw_tile = take((size_t)l.n_tiles * BH * (size_t)fines * D * 4);
  l.dsw = take(BH * (size_t)fines * D * 4);
  l.dpz = take(BH * (size_t)st->page_cap * D * 4);
  l.dz = take(BH * (size_t)fines * D * 4);
  const bool feat = feature_writer(st) && fines > 0;
  const size_t pages =
      ((assoc_writer(st) || feat) && st->page_c) ? (size_t)fines / st->coarse_group : 0;
  l.dpc = take(BH * pages * D * D * 4);
  l.dalpha = take(4);
  l.zero_end = off;
  l.dalpha_parts = take((size_t)tao::fuse_bwd_workgroups((int)T, (int)B, (int)H) * 4);
  if ((assoc_writer(st) || feat) && fines > 0) {
    const size_t mats = (size_t)fines * BH, mat = D * D * 4;
    l.stats = take(2 * mats * mat);
    l.sol_y = take(mats * mat);
    l.sol_w = take(mats * mat);
    l.sgram = take(mats * mat);
    l.dk_extra = take(rows * D * 4);
    l.starts = take((size_t)fines * 8);
    const size_t pmats = pages * BH;
    l.pstats = take(2 * pmats * mat);
    l.psol_y = take(pmats * mat);
    l.psol_w = take(pmats * mat);
    l.psgram = take(pmats * mat);
    if (feat) {
      const size_t vec = mats * D * 4, pvec = pmats * D * 4;
      l.pstats = take(2 * pmats * mat + 2 * pvec);   // also square, cross, mass sums
      l.fmass = take(vec);
      l.fdmass = take(vec);
      l.fdsq = take(vec);
      l.fdms = take(vec);
      l.fdz = take(vec);
      l.fdpz = take(pvec);
      l.wv = take(rows * tao::kMixMaxRank * 4);
      l.dmv = take(rows * tao::kMixMaxRank * 4);
      l.pdsq = take(pvec);
      l.pdms = take(pvec);
    }
  }
  l.total = off;
  return l;
}

// The feature writers' mixture reads backward (mix_bwd.hip): d C^T and d z
// of the fines from d fine (the fusion adjoint's dnum, den being 1) and, with
// page values, of the completed pages from d coarse; dh accumulates both.
hipError_t feature_read_backward(const tao_state_dev* st, const tao_prefill_pools* pools,
                                 const TrainBwdLayout& l, char* ws, const tao::MemBwdParams& mp,
                                 const tao::TrainBwdParams& fp, int fines, int T,
                                 hipStream_t s) {
  const int B = st->batch, H = st->heads, D = st->head_dim, G = st->coarse_group;
  hipError_t e = hipMemsetAsync(mp.dh, 0, (size_t)B * T * H * D * sizeof(float), s);
  if (e != hipSuccess) return e;
  tao::MixBwdParams mx{};
  mx.h = fp.h;
  mx.dout = fp.dnum;
  mx.z = (const bf16_t*)st->fine_z;
  mx.mats = (const bf16_t*)st->bank_c;
  mx.cap = st->fine_cap;
  mx.qsel = pools->qsel;
  mx.qsel_words = pools->qsel_words;
  mx.dh = mp.dh;
  mx.wv = (float*)(ws + l.wv);
  mx.dmv = (float*)(ws + l.dmv);
  mx.R = tao::kMixMaxRank;
  mx.dmat = mp.dc;
  mx.dz = (float*)(ws + l.fdz);
  mx.n_items = fines;
  mx.B = B;
  mx.H = H;
  mx.T = T;
  mx.ft = st->fine_tokens;
  mx.keep = st->local_keep;
  mx.group = G;
  mx.first_query = st->local_keep + st->fine_tokens;
  e = tao::launch_mix_bwd(mx, D, s);
  if (e != hipSuccess || !st->page_c || fines / G < 1) return e;
  tao::MixBwdParams mc = mx;
  mc.dout = fp.dcoarse;
  mc.z = (const bf16_t*)st->page_z;
  mc.mats = (const bf16_t*)st->page_c;
  mc.cap = st->page_cap;
  mc.qsel = nullptr;
  mc.qsel_words = 0;
  mc.dmat = (float*)(ws + l.dpc);
  mc.dz = (float*)(ws + l.fdpz);
  mc.n_items = fines / G;
  mc.first_query = st->local_keep + G * st->fine_tokens;
  return tao::launch_mix_bwd(mc, D, s);
}

}  // namespace

size_t tao_train_bwd_workspace_bytes(const tao_state_dev* st, int64_t tokens, int32_t fines,
                                     const tao_prefill_pools* pools) {
  if (!st || tokens < 0 || fines < 0) return 0;
  return train_bwd_layout(st, tokens, fines, pools).total;
}

int tao_train_backward(const tao_state_dev* st, const tao_tokens* tok, const tao_fusion* fu,
                       const tao_prefill_pools* pools, const tao_train_bwd* a, void* stream) {
  int rc = check_state(st);
  if (!rc) rc = check_tokens(tok);
  if (!rc) rc = check_fusion(fu);
  if (rc) return rc;
  if (!a || !a->grad || !a->local || !a->dv || !a->draw_q || !a->draw_k || !a->dfusion_a ||
      !a->dfusion_b || !a->workspace)
    return fail(TAO_E_ARGUMENT, "null backward argument");
  const bool plugin_local = a->dlocal_out != nullptr;
  if (!plugin_local && (!a->local_lse || !a->dq || !a->dk))
    return fail(TAO_E_ARGUMENT, "null local-attention save or gradient");
  const int T = tok->tokens;
  const int ft = st->fine_tokens, keep = st->local_keep, G = st->coarse_group;
  const int n_tiles = (T + ft - 1) / ft;
  const int lag = keep / ft;
  const int fines = n_tiles - 1 - lag > 0 ? n_tiles - 1 - lag : 0;
  if (fines > 0) {
    if (!pools || !pools->pw_pool || !pools->psw_pool || !pools->qsel || !a->coarse_out ||
        !a->fine_out || !a->den_out)
      return fail(TAO_E_ARGUMENT, "backward with history needs the forward's pools and saves");
    if (fines > st->fine_cap || pools->epochs < fines || pools->pool_pcap < fines / G + 1 ||
        (fines + 31) / 32 > pools->qsel_words)
      return fail(TAO_E_CAPACITY, "backward pools smaller than the full-sequence plan");
    if (fines / G + 1 > 64)
      return fail(TAO_E_CAPACITY, "backward supports at most 63 completed pages (504 fines)");
    if (st->page_c && (fines / G >= 1) &&
        (!pools->coarse_pool || pools->coarse_first != 1 || pools->coarse_count != fines / G))
      return fail(TAO_E_ARGUMENT, "backward with coarse values needs the forward's coarse pool");
  }
  const TrainBwdLayout l = train_bwd_layout(st, T, fines, fines > 0 ? pools : nullptr);
  if (a->workspace_bytes < l.total) return fail(TAO_E_WORKSPACE, "backward workspace too small");
  const bool regularized = assoc_writer(st) && fines > 0;
  const bool featured = feature_writer(st) && fines > 0;
  const hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)a->workspace;
  const int D = st->head_dim, H = st->heads, B = st->batch;
  hipError_t e = hipMemsetAsync(ws + l.zero_begin, 0, l.zero_end - l.zero_begin, s);
  if (e != hipSuccess) return check_hip(e, "tao_train_backward clear");
  // ---- fusion adjoint
  tao::TrainBwdParams fp{};
  fp.grad = (const bf16_t*)a->grad;
  fp.g_sb = a->grad_s[0];
  fp.g_st = a->grad_s[1];
  fp.g_sh = a->grad_s[2];
  fp.rq = view(tok->raw_q, tok->rq_s);
  fp.local = (const bf16_t*)a->local;
  fp.coarse = (const bf16_t*)a->coarse_out;
  fp.fine = (const bf16_t*)a->fine_out;
  fp.den = a->den_out;
  fp.fa = fu->fusion_a;
  fp.fb = fu->fusion_b;
  fp.f_dtype = fu->dtype;
  for (int i = 0; i < 3; ++i) { fp.fa_s[i] = fu->a_s[i]; fp.fb_s[i] = fu->b_s[i]; }
  fp.gain = fu->gain;
  fp.B = B;
  fp.T = T;
  fp.H = H;
  fp.first_fine = keep + ft;
  fp.first_coarse = keep + G * ft;
  fp.coarse_values = st->page_c != nullptr;
  fp.dlocal = (bf16_t*)(ws + l.dlocal);
  fp.delta = (float*)(ws + l.delta);
  fp.dcoarse = (float*)(ws + l.dcoarse);
  fp.dnum = (float*)(ws + l.dnum);
  fp.dden = (float*)(ws + l.dden);
  fp.drq = (float*)(ws + l.drq);
  fp.dfa = a->dfusion_a;
  fp.dfb = a->dfusion_b;
  fp.h = (bf16_t*)(ws + l.h);
  fp.dalpha = (float*)(ws + l.dalpha);
  fp.dalpha_parts = a->dalpha_out ? (float*)(ws + l.dalpha_parts) : nullptr;
  e = tao::launch_fuse_bwd(fp, D, s);
  if (e != hipSuccess) return check_hip(e, "tao_train_backward fusion");
  // ---- local attention adjoint (or d local for the caller's plugin)
  if (plugin_local) {
    e = hipMemcpyAsync(a->dlocal_out, fp.dlocal, (size_t)B * T * H * D * sizeof(bf16_t),
                       hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess)
      e = hipMemsetAsync(ws + l.dvf, 0, (size_t)B * T * H * D * sizeof(float), s);
    if (e != hipSuccess) return check_hip(e, "tao_train_backward d local");
  }
  tao::AttnBwdParams ap{};
  ap.q = view(tok->q, tok->q_s);
  ap.k = view(tok->k, tok->k_s);
  ap.v = view(tok->v, tok->v_s);
  ap.dout = fp.dlocal;
  ap.lse = a->local_lse;
  ap.delta = fp.delta;
  ap.dq = (bf16_t*)a->dq;
  ap.dk = (bf16_t*)a->dk;
  ap.dv = (float*)(ws + l.dvf);
  ap.B = B;
  ap.H = H;
  ap.T = T;
  ap.ft = ft;
  ap.keep = keep;
  e = plugin_local ? hipSuccess : tao::launch_attn_bwd(ap, D, s);
  if (e != hipSuccess) return check_hip(e, "tao_train_backward local attention");
  // ---- memory branch, writer, final gradients
  tao::MemBwdParams mp{};
  mp.bank = (const bf16_t*)st->bank_c;
  mp.fine_sw = (const bf16_t*)st->fine_sw;
  mp.page_z = (const bf16_t*)st->page_z;
  mp.page_c = (const bf16_t*)st->page_c;
  if (fines > 0) {
    mp.pw_pool = (const bf16_t*)pools->pw_pool;
    mp.psw_pool = (const bf16_t*)pools->psw_pool;
    mp.pool_pcap = pools->pool_pcap;
    mp.coarse_pool = (const bf16_t*)pools->coarse_pool;
    mp.coarse_first = pools->coarse_first;
    mp.coarse_count = st->page_c ? pools->coarse_count : 0;
    mp.qsel = pools->qsel;
    mp.qsel_words = pools->qsel_words;
  }
  mp.raw_k = view(tok->raw_k, tok->rk_s);
  mp.v = view(tok->v, tok->v_s);
  mp.h = fp.h;
  mp.dnum = fp.dnum;
  mp.dden = fp.dden;
  mp.dcoarse = fp.dcoarse;
  mp.drq_fuse = fp.drq;
  mp.dh = (float*)(ws + l.dh);
  mp.dpw = (float*)(ws + l.dpw);
  mp.dsw_tile = (float*)(ws + l.dsw_tile);
  mp.dgc = (float*)(ws + l.dgc);
  mp.dc = (float*)(ws + l.dc);
  mp.dsw = (float*)(ws + l.dsw);
  mp.dpz = (float*)(ws + l.dpz);
  mp.dz = (float*)(ws + l.dz);
  mp.dv = ap.dv;
  mp.draw_q = (bf16_t*)a->draw_q;
  mp.draw_k = (bf16_t*)a->draw_k;
  mp.dv_out = (bf16_t*)a->dv;
  mp.B = B;
  mp.H = H;
  mp.T = T;
  mp.ft = ft;
  mp.keep = keep;
  mp.group = G;
  mp.fine_cap = st->fine_cap;
  mp.page_cap = st->page_cap;
  mp.v_max = fines;
  mp.coarse_values = st->page_c != nullptr;
  if (regularized) {
    mp.values_external = 1;
    mp.dpc = (float*)(ws + l.dpc);
    mp.dpc_cap = st->page_c ? fines / G : 0;
  }
  if (featured) {
    e = feature_read_backward(st, pools, l, ws, mp, fp, fines, (int)T, s);
    if (e != hipSuccess) return check_hip(e, "tao_train_backward mixture reads");
    const int pages = st->page_c ? fines / G : 0;
    if (st->fine_writer == TAO_WRITER_FEATURE_MASS) {
      AssocPages pg{l.pstats, l.psol_y, l.psol_w, l.psgram, (const float*)(ws + l.dpc), pages};
      FeatureMass fm{(float*)(ws + l.fmass), (float*)(ws + l.fdmass),
                     (const float*)(ws + l.fdz), (const float*)(ws + l.fdpz), pages};
      e = assoc_backward(st, tok, ws, l.stats, l.sol_y, l.sol_w, l.sgram, l.dk_extra, l.starts,
                         mp.dc, mp.dv, fines, (int)T, pg, s, &fm);
    } else {
      StructuredWs o{l.stats, l.fmass, l.sol_w, l.sgram, l.fdsq, l.fdms, l.fdmass,
                     l.pstats, l.psol_w, l.pdsq, l.pdms};
      e = structured_backward(st, tok, ws, o, l.dk_extra, l.starts, mp.dc,
                              (const float*)(ws + l.dpc), (const float*)(ws + l.fdz),
                              (const float*)(ws + l.fdpz), mp.dv, fines, pages, (int)T, s);
    }
    if (e != hipSuccess) return check_hip(e, "tao_train_backward feature writer");
    mp.values_external = 1;
    mp.dk_extra = (const float*)(ws + l.dk_extra);
  } else {
    e = tao::launch_mem_bwd_read(mp, D, s);
  }
  if (e != hipSuccess) return check_hip(e, "tao_train_backward memory branch");
  if (regularized) {
    AssocPages pg{l.pstats, l.psol_y, l.psol_w, l.psgram, mp.dpc, mp.dpc_cap};
    e = assoc_backward(st, tok, ws, l.stats, l.sol_y, l.sol_w, l.sgram, l.dk_extra, l.starts,
                       mp.dc, mp.dv, fines, (int)T, pg, s);
    if (e != hipSuccess) return check_hip(e, "tao_train_backward association writer");
    mp.dk_extra = (const float*)(ws + l.dk_extra);
  }
  e = tao::launch_mem_bwd_writer(mp, D, s);
  if (e != hipSuccess) return check_hip(e, "tao_train_backward writer branch");
  const size_t BHf = (size_t)B * H * fines;
  if (a->dz_out && fines > 0) {
    const void* dz = featured ? (const void*)(ws + l.fdz) : (const void*)mp.dz;
    e = hipMemcpyAsync(a->dz_out, dz, BHf * D * sizeof(float), hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return check_hip(e, "tao_train_backward dz copy");
  }
  if (a->dc_out && fines > 0) {
    e = hipMemcpyAsync(a->dc_out, mp.dc, BHf * D * D * sizeof(float), hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return check_hip(e, "tao_train_backward dC copy");
  }
  if (a->dalpha_out) {
    e = hipMemcpyAsync(a->dalpha_out, ws + l.dalpha, sizeof(float), hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return check_hip(e, "tao_train_backward d alpha copy");
  }
  return TAO_OK;
}

// ---- non-preset fine writers and the channel-given selected read

namespace {

bool head_ok(int32_t d) { return d == 64 || d == 128; }

void copy3(int64_t dst[3], const int64_t* src) {
  for (int i = 0; i < 3; ++i) dst[i] = src[i];
}

}  // namespace

int tao_writer_statistics(const void* k, const int64_t* k_s, const void* v, const int64_t* v_s,
                          int32_t blocks, int32_t tokens, int32_t heads, int32_t head_dim,
                          int32_t mode, float* gram, float* cross, float* mass, void* stream) {
  if (!head_ok(head_dim)) return fail(TAO_E_SHAPE, "head_dim must be 64 or 128 on the HIP path");
  if (blocks < 0 || tokens < 0 || heads < 0) return fail(TAO_E_SHAPE, "negative extent");
  if (mode != TAO_STATS_ASSOCIATION && mode != TAO_STATS_STRUCTURED)
    return fail(TAO_E_ARGUMENT, "unknown statistics mode");
  if ((size_t)blocks * heads == 0) return TAO_OK;
  if (!k || !v || !k_s || !v_s || !gram || !cross || (mode == TAO_STATS_STRUCTURED && !mass))
    return fail(TAO_E_ARGUMENT, "null operand");
  if (tokens == 0) return fail(TAO_E_SHAPE, "statistics of an empty block");
  tao::WriterStatsParams p{};
  p.k = (const bf16_t*)k;
  p.v = (const bf16_t*)v;
  copy3(p.k_s, k_s);
  copy3(p.v_s, v_s);
  p.N = blocks;
  p.T = tokens;
  p.H = heads;
  p.mode = mode == TAO_STATS_STRUCTURED ? 1 : 0;
  p.gram = gram;
  p.cross = cross;
  p.mass = mass;
  return check_hip(tao::launch_writer_stats(p, head_dim, (hipStream_t)stream),
                   "tao_writer_statistics");
}

int tao_association_matrix(const float* gram, const float* cross, int32_t count, int32_t head_dim,
                           void* out, int32_t* info, void* stream) {
  if (!head_ok(head_dim)) return fail(TAO_E_SHAPE, "head_dim must be 64 or 128 on the HIP path");
  if (count < 0) return fail(TAO_E_SHAPE, "negative count");
  if (count == 0) return TAO_OK;
  if (!gram || !cross || !out) return fail(TAO_E_ARGUMENT, "null operand");
  tao::AssocSolveParams p{};
  p.gram = gram;
  p.cross = cross;
  p.count = count;
  p.out = (bf16_t*)out;
  p.info = info;
  return check_hip(tao::launch_association_solve(p, head_dim, (hipStream_t)stream),
                   "tao_association_matrix");
}

int tao_structured_matrix(const float* square_mass, const float* cross, const float* mass,
                          int32_t count, int32_t head_dim, float tokens, void* out, void* stream) {
  if (!head_ok(head_dim)) return fail(TAO_E_SHAPE, "head_dim must be 64 or 128 on the HIP path");
  if (count < 0) return fail(TAO_E_SHAPE, "negative count");
  if (count == 0) return TAO_OK;
  if (!square_mass || !cross || !mass || !out) return fail(TAO_E_ARGUMENT, "null operand");
  tao::StructuredParams p{};
  p.square = square_mass;
  p.cross = cross;
  p.mass = mass;
  p.count_mats = count;
  p.count = tokens;
  p.out = (bf16_t*)out;
  return check_hip(tao::launch_structured_matrix(p, head_dim, (hipStream_t)stream),
                   "tao_structured_matrix");
}

int tao_chronological_sum(const float* statistics, int64_t outer, int32_t fines, int64_t inner,
                          float* out, void* stream) {
  if (outer < 0 || inner < 0 || fines < 1) return fail(TAO_E_SHAPE, "bad extents");
  if (outer * inner == 0) return TAO_OK;
  if (!statistics || !out) return fail(TAO_E_ARGUMENT, "null operand");
  return check_hip(tao::launch_chrono_sum(statistics, out, outer, fines, inner, (hipStream_t)stream),
                   "tao_chronological_sum");
}

int tao_feature_read_coefficients(const void* h, const int64_t* h_s, const void* read_z,
                                  const int64_t* z_s, int32_t batch, int32_t tokens,
                                  int32_t heads, int32_t pages, int32_t head_dim, void* out,
                                  void* stream) {
  if (!head_ok(head_dim)) return fail(TAO_E_SHAPE, "head_dim must be 64 or 128 on the HIP path");
  if (batch < 0 || tokens < 0 || heads < 0 || pages < 0) return fail(TAO_E_SHAPE, "negative extent");
  if ((size_t)batch * tokens * heads * pages == 0) return TAO_OK;
  if (!h || !h_s || !read_z || !z_s || !out) return fail(TAO_E_ARGUMENT, "null operand");
  tao::FeatureCoeffParams p{};
  p.h = (const bf16_t*)h;
  p.z = (const bf16_t*)read_z;
  copy3(p.h_s, h_s);
  for (int i = 0; i < 4; ++i) p.z_s[i] = z_s[i];
  p.B = batch;
  p.T = tokens;
  p.H = heads;
  p.P = pages;
  p.out = (bf16_t*)out;
  return check_hip(tao::launch_feature_coeff(p, head_dim, (hipStream_t)stream),
                   "tao_feature_read_coefficients");
}

namespace {

int selected_args(tao::SelectedParams& p, const void* channel, const int64_t* selected_id,
                  const void* fine_c, int32_t batch, int32_t queries, int32_t heads,
                  int32_t selected, int32_t bank_batch, int32_t fines, int32_t head_dim) {
  if (!head_ok(head_dim)) return fail(TAO_E_SHAPE, "head_dim must be 64 or 128 on the HIP path");
  if (batch < 0 || queries < 0 || heads < 0 || selected < 0 || fines < 0)
    return fail(TAO_E_SHAPE, "negative extent");
  if (bank_batch < 1 || batch % bank_batch != 0)
    return fail(TAO_E_SHAPE, "batch must be a multiple of the bank batch");
  if (selected > 64) return fail(TAO_E_CAPACITY, "more than 64 selected fines per query");
  if (fines > 4096) return fail(TAO_E_CAPACITY, "more than 4096 fines in the bank");
  if (!channel || !selected_id || !fine_c) return fail(TAO_E_ARGUMENT, "null operand");
  p.channel = (const bf16_t*)channel;
  p.ids = selected_id;
  p.bank = (const bf16_t*)fine_c;
  p.B = batch;
  p.Q = queries;
  p.H = heads;
  p.M = selected;
  p.BB = bank_batch;
  p.S = fines;
  return TAO_OK;
}

}  // namespace

int tao_selected_numerator(const void* channel, const int64_t* selected_id, const void* fine_c,
                           int32_t batch, int32_t queries, int32_t heads, int32_t selected,
                           int32_t bank_batch, int32_t fines, int32_t head_dim, void* out,
                           void* stream) {
  tao::SelectedParams p{};
  const int rc = selected_args(p, channel, selected_id, fine_c, batch, queries, heads, selected,
                               bank_batch, fines, head_dim);
  if (rc) return rc;
  if (!out) return fail(TAO_E_ARGUMENT, "null output");
  p.out = (bf16_t*)out;
  return check_hip(tao::launch_selected_numerator(p, head_dim, (hipStream_t)stream),
                   "tao_selected_numerator");
}

int tao_selected_numerator_backward(const void* channel, const int64_t* selected_id,
                                    const void* fine_c, const void* grad, int32_t batch,
                                    int32_t queries, int32_t heads, int32_t selected,
                                    int32_t bank_batch, int32_t fines, int32_t head_dim,
                                    void* grad_channel, void* grad_fine_c, void* stream) {
  tao::SelectedParams p{};
  const int rc = selected_args(p, channel, selected_id, fine_c, batch, queries, heads, selected,
                               bank_batch, fines, head_dim);
  if (rc) return rc;
  if (!grad) return fail(TAO_E_ARGUMENT, "null gradient");
  p.grad = (const bf16_t*)grad;
  p.grad_channel = (bf16_t*)grad_channel;
  p.grad_bank = (bf16_t*)grad_fine_c;
  return check_hip(tao::launch_selected_numerator_bwd(p, head_dim, (hipStream_t)stream),
                   "tao_selected_numerator_backward");
}

