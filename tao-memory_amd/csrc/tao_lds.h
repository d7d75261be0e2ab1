// LDS streaming helpers for gfx950 kernels that fill LDS with direct
// global-to-LDS copies (global_load_lds_dwordx4).
//
// The compiler does not order such copies against its own LDS accesses, so
// kernels that keep copies in flight while they compute read the staged
// data with the explicit ds_read instructions below and wait for them
// themselves: s_waitcnt vmcnt for their copies (before the barrier that
// publishes them), s_waitcnt lgkmcnt for their reads. A value read this way
// is ready only after its wait, so every use must be tied to the wait
// (wait_lgkm's operand, or after_waits after it): the compiler treats an
// asm output as available at once.
#pragma once

#include <type_traits>
#include <utility>

#include "tao_common.h"

namespace tao {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;

TAO_DEV bf16x8 as_bf16x8(const uint4& u) {
  bf16x8 r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

TAO_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// 16 bytes from LDS byte address addr + OFF, not waited for.
template <int OFF>
TAO_DEV u32x4 ds_read16(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

// Transposing 8-byte LDS read (ds_read_b64_tr_b16), not waited for. Within
// each 16 lanes, lane i receives element i % 4 of the 8 bytes that lane
// 4k + i / 4 addresses, for k = 0..3: lanes that address a 4-row x
// 16-column tile of 16-bit elements (lane s: row s / 4, columns
// 4 (s % 4) .. + 3) each receive the 4 rows of one column.
template <int OFF>
TAO_DEV u32x2 ds_read_tr8(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

// s_waitcnt lgkmcnt(N), tied to the values it makes ready (nothing that
// reads them is scheduled above it).
template <int N, typename T>
TAO_DEV void wait_lgkm(T& a) {
  static_assert(N >= 0 && N < 16, "lgkmcnt is four bits");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "i"(N) : "memory");
}

// Ties a value to the waits issued before it: an empty volatile statement
// stays after them, and every use of the value after it.
template <typename T>
TAO_DEV void after_waits(T& a) { asm volatile("" : "+v"(a)); }

TAO_DEV void wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// s_waitcnt lgkmcnt(0) for this wave's own LDS writes (before a barrier).
TAO_DEV void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>), in order.
template <typename F, int... I>
TAO_DEV void unroll_seq(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>()), ...);
}
template <int N, typename F>
TAO_DEV void unroll(F&& f) {
  unroll_seq(f, std::make_integer_sequence<int, N>());
}


// 4 bytes from / to LDS byte address addr + OFF, not waited for.
template <int OFF>
TAO_DEV float ds_read4(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  float r;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int OFF>
TAO_DEV void ds_write4(uint32_t addr, float v) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  asm volatile("ds_write_b32 %0, %1 offset:%2" : : "v"(addr), "v"(v), "i"(OFF) : "memory");
}

// s_waitcnt vmcnt(N): every copy or load of this wave but the newest N has
// landed (expcnt and lgkmcnt not waited for).
template <int N>
TAO_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  asm volatile("s_waitcnt vmcnt(%0)" : : "i"(N) : "memory");
}

// 16 bytes to LDS byte address addr + OFF, not waited for.
template <int OFF>
TAO_DEV void ds_write16(uint32_t addr, const u32x4& v) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "i"(OFF) : "memory");
}

}  // namespace tao
