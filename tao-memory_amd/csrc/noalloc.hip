// tao_decode_step_noalloc: the single-token decode step for callers that
// cannot allocate device memory (code under graph capture, tight serving
// loops, harnesses that forbid hipMalloc). It runs the same kernel as
// tao_decode_step; only the step's per-head records and its arrival
// counters move from the state's workspace into two file-scope device
// arrays of fixed size, so the caller's state needs no workspace at all.
//
// The arrays hold kScratchBytes and kMaxCounters counters per device for the
// life of the process. Their addresses are resolved once per device with
// hipGetSymbolAddress (with that device current) and kept; host code passes
// those addresses, never the arrays' names, to the kernel. Every call on one
// device shares them: calls that overlap on one device (two streams, two
// host threads) race and must be serialised by the caller. The records need
// no initial value (each step writes every record it reads; an empty local
// record carries l = 0). The counters must be zero between steps: device
// arrays start zeroed when the library loads, and every step's last arrival
// resets each counter it used.
#include <mutex>
#include <string>

#include "tao_launch.h"

namespace {

constexpr size_t kScratchBytes = size_t(4) << 20;   // 4 MiB per device
constexpr int kMaxCounters = 1024;                   // heads + 1 per step
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
static __device__ __align__(256) unsigned scratch_counters[kMaxCounters * tao::kCounterStride];

std::mutex g_scratch_lock;
float* g_scratch[kMaxDevices] = {};
unsigned* g_counters[kMaxDevices] = {};

int fail(int code, const std::string& msg) {
  tao::set_error(msg.c_str());
  return code;
}

// The current device's copies of `scratch` and `scratch_counters` (resolved
// on the first call there).
int device_scratch(float** out, unsigned** counters) {
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
    void* cptr = nullptr;
    e = hipGetSymbolAddress(&cptr, HIP_SYMBOL(scratch_counters));
    if (e != hipSuccess || !cptr)
      return fail(e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol,
                  std::string("tao_decode_step_noalloc: hipGetSymbolAddress: ") +
                      hipGetErrorString(e));
    g_scratch[dev] = (float*)ptr;
    g_counters[dev] = (unsigned*)cptr;
  }
  *out = g_scratch[dev];
  *counters = g_counters[dev];
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
                    "-byte static scratch (at most 467 heads at D128, 531 at D64)");
  if (tao::step_counters(st->batch, st->heads) > (size_t)kMaxCounters)
    return fail(TAO_E_CAPACITY, "tao_decode_step_noalloc: more heads than the static "
                                "scratch counts");
  float* records = nullptr;
  unsigned* counters = nullptr;
  const int rc = device_scratch(&records, &counters);
  if (rc) return rc;
  return tao::decode_step_at(st, tok, fu, selected, out, out_s, stream, -1, records, counters);
}
