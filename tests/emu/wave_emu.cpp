// wave_emu.cpp -- runs the engine's per-position programs (hive_phases.hpp)
// on the host, one emulated 64-lane wave per call.  TEST INFRASTRUCTURE ONLY:
// used by tests/test_emu_engine.py to check the device logic on the CPU and
// to debug it there.
#define HW_HOST_EMU 1
#include <memory>
#include <thread>
#include <vector>

#include "../../hive_neuralnet_amd/csrc/hive_phases.hpp"

using namespace hw;

namespace {
// Runs body(i, tid) for i in [0, count) on one emulated workgroup of
// `threads` threads (2 positions per 64), one item after another.
template <typename F>
void run_group(int threads, int64_t count, F&& body) {
    std::barrier<> wg(threads);
    std::vector<std::unique_ptr<std::barrier<>>> groups;
    wave_emu::Ctx ctx;
    for (int g = 0; g < threads / wave_emu::kGroupLanes; g++) {
        groups.emplace_back(new std::barrier<>(wave_emu::kGroupLanes));
        ctx.group_bar[g] = groups.back().get();
    }
    ctx.wg_bar = &wg;
    wave_emu::g_ctx = &ctx;
    std::vector<std::thread> th;
    for (int t = 0; t < threads; t++) {
        th.emplace_back([&, t] {
            wave_emu::g_tid = t;
            for (int64_t i = 0; i < count; i++) {
                body(i, t);
                wave_emu::wg_sync();
            }
        });
    }
    for (auto& x : th) x.join();
    wave_emu::g_ctx = nullptr;
}
static Pos g_pos[kPosPerWave];
}  // namespace

extern "C" {
// one emulated wave per kPosPerWave items, as the kernels launch them
void emu_legal(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* n, float* feat, int32_t* act) {
    run_group(64, (B + kPosPerWave - 1) / kPosPerWave, [&](int64_t w, int t) {
        int64_t i = w * kPosPerWave + t / kW;
        bool live = i < B;
        if (!live) i = B - 1;
        run_legal<true, true, true>(g_pos[t / kW], states + i * kStateBytes, t, live ? moves + i * 1536 : nullptr,
                                    live ? n + i : nullptr, live ? feat + i * kFeat : nullptr,
                                    live ? act + i * kMaxLegal : nullptr);
    });
}
void emu_successor(const uint8_t* states, const uint8_t* legal, const int64_t* a2r, const int64_t* midx, int64_t N,
                   float* feat) {
    run_group(64, (N + kPosPerWave - 1) / kPosPerWave, [&](int64_t w, int t) {
        int64_t i = w * kPosPerWave + t / kW;
        bool live = i < N;
        if (!live) i = N - 1;
        run_successor(g_pos[t / kW], states + a2r[i] * kStateBytes, legal + (a2r[i] * kMaxLegal + midx[i]) * 6, t,
                      live ? feat + i * kFeat : nullptr);
    });
}
void emu_queen_escape(const uint8_t* states, int64_t B, uint8_t* out) {
    run_group(64, (B + kPosPerWave - 1) / kPosPerWave, [&](int64_t w, int t) {
        int64_t i = w * kPosPerWave + t / kW;
        bool live = i < B;
        if (!live) i = B - 1;
        bool e = run_queen_escape(g_pos[t / kW], states + i * kStateBytes, t);
        if (live && t % kW == 0) out[i] = e ? 1 : 0;
    });
}
}
