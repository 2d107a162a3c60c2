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
template <typename F>
void run_wave(int64_t count, F&& body) {
    std::barrier<> bar(64);
    wave_emu::Ctx ctx;
    ctx.bar = &bar;
    wave_emu::g_ctx = &ctx;
    static Pos P;
    std::vector<std::thread> lanes;
    for (int l = 0; l < 64; l++) {
        lanes.emplace_back([&, l] {
            wave_emu::g_lane = l;
            for (int64_t i = 0; i < count; i++) {
                body(P, i, l);
                wave_emu::sync();
            }
        });
    }
    for (auto& t : lanes) t.join();
    wave_emu::g_ctx = nullptr;
}
}  // namespace

extern "C" {
void emu_legal(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* n, float* feat, int32_t* act) {
    run_wave(B, [&](Pos& P, int64_t i, int l) {
        run_legal<true, true, true>(P, states + i * kStateBytes, l, moves + i * 1536, n + i, feat + i * kFeat,
                                    act + i * kMaxLegal);
    });
}
void emu_successor(const uint8_t* states, const uint8_t* legal, const int64_t* a2r, const int64_t* midx, int64_t N,
                   float* feat) {
    run_wave(N, [&](Pos& P, int64_t i, int l) {
        run_successor(P, states + a2r[i] * kStateBytes, legal + (a2r[i] * kMaxLegal + midx[i]) * 6, l,
                      feat + i * kFeat);
    });
}
void emu_queen_escape(const uint8_t* states, int64_t B, uint8_t* out) {
    run_wave(B, [&](Pos& P, int64_t i, int l) {
        bool e = run_queen_escape(P, states + i * kStateBytes, l);
        if (l == 0) out[i] = e ? 1 : 0;
    });
}
}
