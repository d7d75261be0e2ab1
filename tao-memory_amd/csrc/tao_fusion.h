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

}  // namespace tao
