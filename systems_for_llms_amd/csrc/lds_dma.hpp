// Buffer loads that write LDS directly (gfx950 "load to LDS"), shared by the
// prefill GEMM and the masked attention.
//
// One 16-byte-per-lane buffer load with an LDS destination: lane i's bytes
// land at LDS byte offset lds + 16 i (M0 holds the wave-uniform base). Written
// as inline assembly because the compiler, unable to tell LDS-DMA targets
// apart, otherwise waits for every outstanding load before each LDS read,
// which serialises the prefetch; the caller therefore counts these loads
// itself (s_waitcnt vmcnt). Loads the compiler does not know about only make
// its own vmcnt waits stricter, never looser. Out-of-range offsets read zeros
// (buffer range check).
#pragma once
#include "common.hpp"

namespace sfl {

typedef int i32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4_t buffer_rsrc(const void* base, unsigned bytes) {
  const unsigned long long b = reinterpret_cast<unsigned long long>(base);
  return i32x4_t{int(b & 0xffffffffu), int(b >> 32), int(bytes), 0x00020000};
}
__device__ __forceinline__ void lds_load16(i32x4_t rsrc, unsigned lds, unsigned voff, unsigned soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(rsrc), "s"(soff) : "memory");
}
__device__ __forceinline__ unsigned lds_offset(const void* p) {
  return unsigned(size_t((__attribute__((address_space(3))) const char*)(p)));
}

// s_waitcnt operand that waits for vmcnt <= n only (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
constexpr int sfl_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

}  // namespace sfl
