// Three-branch presence-aware fusion for one (b, t, h, d) element.
//
// Restates fusion_pointwise.py:10-92 plus the torch softmax between them
// (operator.py:86-94): every intermediate is rounded to bf16 exactly where
// the reference rounds, with no FMA contraction (the reference launches both
// kernels with enable_fp_fusion=False). The branch softmax uses the hardware
// exp and one reciprocal: it only shapes the output (within the bf16
// tolerance), never a routing decision.
#pragma once

#include "tao_common.h"

namespace tao {

// A caller fusion parameter as fp32 (exact for every accepted dtype).
TAO_DEV float load_param(const void* p, int dtype, int64_t off) {
  if (dtype == TAO_FP32) return ((const float*)p)[off];
  if (dtype == TAO_FP16) return (float)((const _Float16*)p)[off];
  return bf2f(((const bf16_t*)p)[off]);
}

// bf16(fp32(log 2)) = 0.69140625: the local bias when two history branches
// are present (fusion_pointwise.py:114-117, operator.py branch count).
constexpr float kLogTwoBf16 = 0.69140625f;

// The branch weights of one channel (fusion_pointwise.py:10-117): they
// depend on the raw query element and the parameters only, not on the
// branch values, so a decode step computes them beside its reads.
struct FuseWeights {
  float r0, r1, r2;   // local, coarse, fine
};

TAO_DEV FuseWeights fuse_weights(float q, const float a[3], const float b[3], int coarse_on,
                                 int fine_on) {
  const float ninf = -__builtin_inff();
  float s[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    float prod = rbf(rbf(a[i]) * q);
    s[i] = rbf(prod + rbf(b[i]));
  }
  float bias = (coarse_on && fine_on) ? kLogTwoBf16 : 0.0f;
  s[0] = rbf(s[0] + bias);
  if (!coarse_on) s[1] = ninf;
  if (!fine_on) s[2] = ninf;
  float top = fmaxf(s[0], fmaxf(s[1], s[2]));
  float e0 = __expf(s[0] - top);
  float e1 = coarse_on ? __expf(s[1] - top) : 0.0f;
  float e2 = fine_on ? __expf(s[2] - top) : 0.0f;
  float total = (e0 + e2) + e1;   // butterfly order over [e0, e1, e2, 0]
  const float inv = __builtin_amdgcn_rcpf(total);
  return {rbf(e0 * inv), rbf(e1 * inv), rbf(e2 * inv)};
}

// The weighted mix of the branch values with the channel's weights.
TAO_DEV bf16_t fuse_mix(const FuseWeights& w, float local, float coarse, float fine, float gain) {
  float lt = rbf(w.r0 * rbf(2.0f * local));
  float ct = rbf(w.r1 * rbf(gain * coarse));
  float ft = rbf(w.r2 * rbf(gain * fine));
  return f2bf(rbf(lt + ct) + ft);
}

TAO_DEV bf16_t fuse_element(float q, float local, float coarse, float fine,
                            const float a[3], const float b[3], float gain,
                            int coarse_on, int fine_on) {
  return fuse_mix(fuse_weights(q, a, b, coarse_on, fine_on), local, coarse, fine, gain);
}

// Rounds x and y to bf16 with one packed conversion.
TAO_DEV void rbf2(float& x, float& y) {
  const uint32_t pk = pack_bf16x2(x, y);
  x = __uint_as_float(pk << 16);
  y = __uint_as_float(pk & 0xFFFF0000u);
}

// Two adjacent channels of the fusion with the fine branch present and the
// coarse branch absent, packed as bf16x2 (channel 0 low). Bit-identical to
// fuse_element(q[j], local[j], 0, fine[j], a[j], b[j], gain, 0, 1) with
// ra = rbf(a), rb = rbf(b): each rounding point is the same, paired over
// the two channels, and the coarse terms are folded. Without the coarse
// branch the local bias is 0, so rbf(s0 + 0) differs from s0 only in the
// sign of a zero, which no later step sees (exp(s - top) is 1 for either
// zero); the coarse weight is +0, so the total is e0 + e2, and the coarse
// term is ct0 = rbf(+0 * rbf(gain * 0)), a signed zero that the caller
// computes once, so rbf(lt + ct) = lt + ct0 (lt is already bf16).
TAO_DEV uint32_t fuse_pair_local_fine(const float q[2], const float local[2], const float fine[2],
                                      const float ra[2][3], const float rb[2][3], float gain,
                                      float ct0) {
  float p0[2], p2[2], e0[2], e2[2], l2[2], gf[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    p0[j] = ra[j][0] * q[j];
    p2[j] = ra[j][2] * q[j];
  }
  rbf2(p0[0], p0[1]);
  rbf2(p2[0], p2[1]);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    p0[j] = p0[j] + rb[j][0];
    p2[j] = p2[j] + rb[j][2];
  }
  rbf2(p0[0], p0[1]);
  rbf2(p2[0], p2[1]);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    // exp(p - top) of the larger branch is exp(0) = 1 exactly, so only the
    // other one's exp is computed (a NaN lands in that exp, so it still
    // makes both weights NaN).
    const bool first = p0[j] >= p2[j];
    const float top = first ? p0[j] : p2[j], low = first ? p2[j] : p0[j];
    const float xl = __expf(low - top);
    const float x0 = first ? 1.0f : xl, x2 = first ? xl : 1.0f;
    const float inv = __builtin_amdgcn_rcpf(x0 + x2);
    e0[j] = x0 * inv;
    e2[j] = x2 * inv;
    l2[j] = 2.0f * local[j];
    gf[j] = gain * fine[j];
  }
  rbf2(e0[0], e0[1]);
  rbf2(e2[0], e2[1]);
  rbf2(l2[0], l2[1]);
  rbf2(gf[0], gf[1]);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    l2[j] = e0[j] * l2[j];
    gf[j] = e2[j] * gf[j];
  }
  rbf2(l2[0], l2[1]);
  rbf2(gf[0], gf[1]);
  return pack_bf16x2((l2[0] + ct0) + gf[0], (l2[1] + ct0) + gf[1]);
}

}  // namespace tao
