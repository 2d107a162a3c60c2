// wave_emu.cpp -- runs the engine's per-position programs (hive_phases.hpp)
// on the host, one emulated 64-lane wave per call.  TEST INFRASTRUCTURE ONLY:
// used by tests/test_emu_engine.py to check the device logic on the CPU and
// to debug it there.
#define HW_HOST_EMU 1
#include <thread>
#include <vector>

#include "../../hive_neuralnet_amd/csrc/hive_phases.hpp"

using namespace hw;

namespace {
// Runs body(i, tid) for i in [0, count) on one emulated workgroup of
// `waves` waves, one item after another.
template <typename F>
void run_group(int waves, int64_t count, F&& body) {
    std::barrier<> gbar(waves * 64);
    std::barrier<> wb0(64), wb1(64), wb2(64), wb3(64);
    wave_emu::Ctx ctx;
    ctx.wave_bar[0] = &wb0; ctx.wave_bar[1] = &wb1; ctx.wave_bar[2] = &wb2; ctx.wave_bar[3] = &wb3;
    ctx.group_bar = &gbar;
    wave_emu::g_ctx = &ctx;
    std::vector<std::thread> threads;
    for (int t = 0; t < waves * 64; t++) {
        threads.emplace_back([&, t] {
            wave_emu::g_tid = t;
            for (int64_t i = 0; i < count; i++) {
                body(i, t);
                wave_emu::group_sync();
            }
        });
    }
    for (auto& th : threads) th.join();
    wave_emu::g_ctx = nullptr;
}
static Pos g_one;
}  // namespace

extern "C" {
void emu_legal(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* n, float* feat, int32_t* act) {
    run_group(1, B, [&](int64_t i, int l) {
        run_legal<true, true, true>(g_one, states + i * kStateBytes, l, moves + i * 1536, n + i, feat + i * kFeat,
                                    act + i * kMaxLegal);
    });
}
void emu_successor(const uint8_t* states, const uint8_t* legal, const int64_t* a2r, const int64_t* midx, int64_t N,
                   float* feat) {
    run_group(1, N, [&](int64_t i, int l) {
        run_successor(g_one, states + a2r[i] * kStateBytes, legal + (a2r[i] * kMaxLegal + midx[i]) * 6, l,
                      feat + i * kFeat);
    });
}
void emu_queen_escape(const uint8_t* states, int64_t B, uint8_t* out) {
    run_group(1, B, [&](int64_t i, int l) {
        bool e = run_queen_escape(g_one, states + i * kStateBytes, l);
        if (l == 0) out[i] = e ? 1 : 0;
    });
}
}
