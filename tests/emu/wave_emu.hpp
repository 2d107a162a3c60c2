// wave_emu.hpp -- host emulation of the few HIP wave primitives the engine
// uses, so tests can run the engine's device code on the CPU.
//
// TEST INFRASTRUCTURE ONLY.  A "wave" is 64 std::threads; barriers, shuffles
// and ballots rendezvous through a shared exchange buffer.  This build never
// ships in the package: the product is the gfx950 HIP library.
#pragma once
#include <atomic>
#include <barrier>
#include <cstdint>
#include <cstdlib>
#include <cstring>

#define __device__
#define __host__
#define __global__
#define __shared__
#define __constant__
#define __forceinline__ inline
#define __launch_bounds__(x)

namespace wave_emu {
// A workgroup of one or more waves.  The engine's cross-lane operations stay
// inside a lane group of kGroupLanes (one position); they rendezvous per
// group, so a group may take a branch the other group of its wave skips.
// __syncthreads synchronises the whole workgroup.
constexpr int kGroupLanes = 32;
struct Ctx {
    std::barrier<>* group_bar[8];
    std::barrier<>* wg_bar;
    int64_t slot[256];
};
inline Ctx* g_ctx = nullptr;
inline thread_local int g_tid = 0;
inline int lane() { return g_tid & 63; }
inline int group() { return g_tid / kGroupLanes; }
inline int group_base() { return g_tid & ~(kGroupLanes - 1); }
inline void group_sync() { g_ctx->group_bar[group()]->arrive_and_wait(); }
inline void wg_sync() { g_ctx->wg_bar->arrive_and_wait(); }
// value of v at wave lane src, which must be in the caller's group
template <typename T>
inline T exchange(T v, int src) {
    int s = (g_tid & ~63) | (src & 63);
    if ((s & ~(kGroupLanes - 1)) != group_base()) abort();
    g_ctx->slot[g_tid] = (int64_t)v;
    group_sync();
    T r = (T)g_ctx->slot[s];
    group_sync();
    return r;
}
}  // namespace wave_emu

struct EmuThreadIdx {
    operator int() const { return wave_emu::g_tid; }
};
struct EmuDim3 {
    EmuThreadIdx x;
};
inline EmuDim3 threadIdx;
struct EmuBlockIdx {
    operator int() const { return 0; }
};

inline void __syncthreads() { wave_emu::wg_sync(); }

template <typename T>
inline T __shfl_up(T v, unsigned o, int = 64) {
    int src = wave_emu::lane() - (int)o;
    return wave_emu::exchange(v, src >= 0 ? src : wave_emu::lane());
}
template <typename T>
inline T __shfl_xor(T v, int m, int = 64) {
    return wave_emu::exchange(v, wave_emu::lane() ^ m);
}
template <typename T>
inline T __shfl(T v, int src, int = 64) {
    return wave_emu::exchange(v, src & 63);
}
// the caller's group bits, at their wave positions
inline uint64_t __ballot(int pred) {
    wave_emu::g_ctx->slot[wave_emu::g_tid] = pred ? 1 : 0;
    wave_emu::group_sync();
    uint64_t m = 0;
    int base = wave_emu::group_base();
    for (int i = 0; i < wave_emu::kGroupLanes; i++)
        if (wave_emu::g_ctx->slot[base + i]) m |= 1ull << ((base & 63) + i);
    wave_emu::group_sync();
    return m;
}
// wave-wide "any": a rendezvous of the whole (one-wave) workgroup
inline bool hw_wave_any(bool p) {
    wave_emu::g_ctx->slot[wave_emu::g_tid] = p ? 1 : 0;
    wave_emu::wg_sync();
    bool any = false;
    for (int i = 0; i < 64; i++) any |= wave_emu::g_ctx->slot[i] != 0;
    wave_emu::wg_sync();
    return any;
}
inline uint32_t __umul24(uint32_t a, uint32_t b) { return (a & 0xFFFFFFu) * (b & 0xFFFFFFu); }
inline uint32_t __builtin_amdgcn_alignbyte(uint32_t hi, uint32_t lo, uint32_t s) {
    return (uint32_t)(((((uint64_t)hi) << 32) | lo) >> (8 * (s & 3)));
}
// DPP lane moves used by the engine's prefix sums: row_shr:1..15, row_bcast:15,
// row_bcast:31 (GFX9 semantics).  Every lane of the wave calls it.
// v_perm_b32: byte k of the result is selected by byte k of sel from the
// 8 bytes {hi:lo} (0-7), or 0x00 for selector 0x0c (the only other value used)
inline uint32_t __builtin_amdgcn_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    uint64_t v = ((uint64_t)hi << 32) | lo;
    uint32_t r = 0;
    for (int k = 0; k < 4; k++) {
        uint32_t b = (sel >> (8 * k)) & 0xFF;
        if (b < 8) r |= (uint32_t)((v >> (8 * b)) & 0xFF) << (8 * k);
        else if (b != 0x0c) abort();
    }
    return r;
}
inline int __builtin_amdgcn_update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    int l = wave_emu::lane(), row = l >> 4, r = l & 15, bank = r >> 2;
    bool enabled = ((row_mask >> row) & 1) && ((bank_mask >> bank) & 1);
    int from = -1;
    if (ctrl >= 0x111 && ctrl <= 0x11F) {
        int n = ctrl - 0x110;
        if (r >= n) from = l - n;
    } else if (ctrl == 0x142) {
        if (row >= 1) from = (row - 1) * 16 + 15;
    } else if (ctrl == 0x143) {
        if (row >= 2) from = 31;
    } else {
        abort();
    }
    if (!enabled) from = -1;
    int v = wave_emu::exchange(src, from >= 0 ? from : l);
    if (!enabled) return old;
    if (from < 0) return bound_ctrl ? 0 : old;
    return v;
}
inline int __builtin_amdgcn_readlane(int v, int l) { return wave_emu::exchange(v, l); }
// v_rcp_f32 is within 1 ulp of 1 / x; the correctly rounded quotient is one such value
inline float __builtin_amdgcn_rcpf(float x) { return 1.0f / x; }
inline int atomicAdd(int* p, int v) { return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }
inline unsigned long long atomicAdd(unsigned long long* p, unsigned long long v) {
    return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST);
}
inline uint32_t atomicOr(uint32_t* p, uint32_t v) { return __atomic_fetch_or(p, v, __ATOMIC_SEQ_CST); }
inline int __popc(uint32_t x) { return __builtin_popcount(x); }
inline int __popcll(uint64_t x) { return __builtin_popcountll(x); }
inline int __ffs(uint32_t x) { return __builtin_ffs((int)x); }
inline int __ffs(int x) { return __builtin_ffs(x); }
inline int __ffsll(unsigned long long x) { return __builtin_ffsll((long long)x); }
inline int __clz(uint32_t x) { return x ? __builtin_clz(x) : 32; }
inline int __clzll(long long x) { return x ? __builtin_clzll((unsigned long long)x) : 64; }
inline uint32_t __umulhi(uint32_t a, uint32_t b) { return (uint32_t)(((uint64_t)a * b) >> 32); }
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
