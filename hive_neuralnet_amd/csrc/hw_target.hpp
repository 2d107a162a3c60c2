// hw_target.hpp -- target header for the wave engine.  The product build is
// HIP for gfx950.  tests/emu compiles the same engine sources for the host
// (HW_HOST_EMU, a 64-thread wave emulator used only by CPU tests and for
// debugging); that build never ships in the package.
#pragma once
#ifdef HW_HOST_EMU
#include "../../tests/emu/wave_emu.hpp"
#else
#include <hip/hip_runtime.h>
#endif

// Every engine routine is inlined into its kernel: a device-side call makes
// the whole kernel allocate for the call ABI (twice the registers, half the
// occupancy of the inlined form for k_legal).
#define HW_INL __device__ __attribute__((always_inline)) inline

// v, opaque to the optimiser: values derived from it inside a loop body are
// recomputed per iteration instead of being hoisted and kept in registers
// across the whole body (which costs occupancy in the large programs)
#ifdef HW_HOST_EMU
inline int hw_opaque(int v) { return v; }
#else
__device__ __forceinline__ int hw_opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}
#endif

// The lanes of a lane group are lanes of one wavefront: they run in lockstep
// and the wavefront's LDS accesses complete in program order, so what one
// lane wrote is seen by every lane's later instructions without a barrier.
// The host emulator runs lanes as threads and synchronises the group here.
#ifdef HW_HOST_EMU
inline void hw_group_lockstep() { wave_emu::group_sync(); }
#else
__device__ __forceinline__ void hw_group_lockstep() {}
#endif

// true in every lane of the wavefront when p holds in any of its lanes
#ifndef HW_HOST_EMU
__device__ __forceinline__ bool hw_wave_any(bool p) { return __ballot(p) != 0; }
#endif

// four dwords loaded or stored together (16-byte access, 4-byte alignment)
#ifdef HW_HOST_EMU
typedef uint32_t u32x4 __attribute__((vector_size(16), aligned(4)));
#else
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
#endif
