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
// A workgroup of up to 4 waves: shuffles and ballots rendezvous per wave,
// __syncthreads across the workgroup.
struct Ctx {
    std::barrier<>* wave_bar[4];
    std::barrier<>* group_bar;
    int64_t slot[256];
};
inline Ctx* g_ctx = nullptr;
inline thread_local int g_tid = 0;
inline int lane() { return g_tid & 63; }
inline int wave() { return g_tid >> 6; }
inline void wave_sync() { g_ctx->wave_bar[wave()]->arrive_and_wait(); }
inline void group_sync() { g_ctx->group_bar->arrive_and_wait(); }
template <typename T>
inline T exchange(T v, int src) {
    g_ctx->slot[g_tid] = (int64_t)v;
    wave_sync();
    T r = (T)g_ctx->slot[(wave() << 6) | (src & 63)];
    wave_sync();
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

inline void __syncthreads() { wave_emu::group_sync(); }

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
inline uint64_t __ballot(int pred) {
    wave_emu::g_ctx->slot[wave_emu::g_tid] = pred ? 1 : 0;
    wave_emu::wave_sync();
    uint64_t m = 0;
    int base = wave_emu::wave() << 6;
    for (int i = 0; i < 64; i++)
        if (wave_emu::g_ctx->slot[base + i]) m |= 1ull << i;
    wave_emu::wave_sync();
    return m;
}
// DPP lane moves used by the engine's prefix sums: row_shr:1..15, row_bcast:15,
// row_bcast:31 (GFX9 semantics).  Every lane of the wave calls it.
inline int __builtin_amdgcn_update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    int l = wave_emu::lane(), row = l >> 4, r = l & 15, bank = r >> 2;
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
    int v = wave_emu::exchange(src, from >= 0 ? from : l);
    if (!((row_mask >> row) & 1) || !((bank_mask >> bank) & 1)) return old;
    if (from < 0) return bound_ctrl ? 0 : old;
    return v;
}
inline int __builtin_amdgcn_readlane(int v, int l) { return wave_emu::exchange(v, l); }
inline int atomicAdd(int* p, int v) { return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }
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
