// tao_decode_step_noalloc: the single-token decode step for callers that
// cannot allocate device memory (code under graph capture, tight serving
// loops, harnesses that forbid hipMalloc). It runs the same two kernels as
// tao_decode_step; only the step's per-head records move from the state's
// workspace into a file-scope device array of fixed size, so the caller's
// state needs no workspace at all.
//
// The array holds kScratchBytes per device for the life of the process. Its
// address is resolved once per device with hipGetSymbolAddress (with that
// device current) and kept; host code passes that address, never the
// array's name, to the kernels. Every call on one device shares the array:
// calls that overlap on one device (two streams, two host threads) race and
// must be serialised by the caller. Nothing in it must start at zero: each
// step writes every record it reads (an empty local record carries l = 0,
// and the combine ignores its values), so the last call's contents are
// harmless.
#include <mutex>
#include <string>

#include "tao_launch.h"

namespace {

constexpr size_t kScratchBytes = size_t(4) << 20;   // 4 MiB per device
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_scratch_lock;
float* g_scratch[kMaxDevices] = {};

int fail(int code, const std::string& msg) {
  tao::set_error(msg.c_str());
  return code;
}

// The current device's copy of `scratch` (resolved on the first call there).
int device_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail((int)e, std::string("tao_decode_step_noalloc: hipGetDevice: ") +
                            hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TAO_E_ARGUMENT, "tao_decode_step_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_lock);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol,
                  std::string("tao_decode_step_noalloc: hipGetSymbolAddress: ") +
                      hipGetErrorString(e));
    g_scratch[dev] = (float*)ptr;
  }
  *out = g_scratch[dev];
  return TAO_OK;
}

}  // namespace

extern "C" int tao_decode_step_noalloc(const tao_state_dev* st, const tao_tokens* tok,
                                       const tao_fusion* fu, int32_t selected, void* out,
                                       const int64_t* out_s, void* stream) {
  if (!st) return fail(TAO_E_ARGUMENT, "null state");
  if (st->head_dim != 64 && st->head_dim != 128)
    return fail(TAO_E_SHAPE, "head_dim must be 64 or 128 on the HIP path");
  if (st->batch <= 0 || st->heads <= 0)
    return fail(TAO_E_SHAPE, "batch and heads must be positive");
  const size_t need =
      (size_t)st->batch * st->heads * tao::step_floats(st->head_dim, st->sel_cap) * sizeof(float);
  if (need > kScratchBytes)
    return fail(TAO_E_CAPACITY,
                "tao_decode_step_noalloc: batch * heads = " +
                    std::to_string((long long)st->batch * st->heads) +
                    " needs " + std::to_string(need) + " bytes of step records, above the " +
                    std::to_string(kScratchBytes) +
                    "-byte static scratch (at most 567 heads at D128, 593 at D64)");
  float* records = nullptr;
  const int rc = device_scratch(&records);
  if (rc) return rc;
  return tao::decode_step_at(st, tok, fu, selected, out, out_s, stream, -1, records);
}
