#include <mutex>
#include <atomic>
// wave_emu.cpp -- runs the engine's per-position programs (hive_phases.hpp)
// on the host, one emulated 64-lane wave per call.  TEST INFRASTRUCTURE ONLY:
// used by tests/test_emu_engine.py to check the device logic on the CPU and
// to debug it there.
#define HW_HOST_EMU 1
#include <memory>
#include <thread>
#include <vector>

#include "../../hive_neuralnet_amd/csrc/hive_probe.hpp"

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
static Replies g_rep[kPosPerWave];
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
// k_successor_features' row streams with blocks of 4 rows and one workgroup
// (each group's stream runs through the blocks 2w + group), the board of a
// run of rows with one root restored from registers
void emu_successor_rows(const uint8_t* states, const uint8_t* legal, const int64_t* a2r, const int64_t* midx,
                        int64_t N, int64_t num_roots, float* feat) {
    static const uint8_t zero_row[kStateBytes] = {};
    const int64_t blocks = (N + 3) / 4;
    static SuccessorStream st[64];
    for (auto& s : st) s = SuccessorStream();
    run_group(64, (blocks + kPosPerWave - 1) / kPosPerWave * 4, [&](int64_t r, int t) {
        int64_t q = (r / 4) * kPosPerWave + t / kW;
        successor_row(g_pos[t / kW], st[t], states, legal, a2r, midx, q * 4 + r % 4, N, num_roots, zero_row, t, feat);
    });
}
// k_random_play's ply loop with given choices: game i's board is loaded
// once, then per ply (while its result is 0) the derived tables are rebuilt,
// the list's tables generated, slot (u[i][ply] * n) >> 32 decoded by
// list_slot and applied by apply_mirrored, which also writes the changed
// bytes into the state row.  done[i]: plies applied.
void emu_play(uint8_t* states, int64_t B, int plies, const uint32_t* u, int32_t* done) {
    run_group(64, (B + kPosPerWave - 1) / kPosPerWave, [&](int64_t w, int t) {
        int64_t i = w * kPosPerWave + t / kW;
        const bool live = i < B;
        if (!live) i = B - 1;
        Pos& P = g_pos[t / kW];
        uint8_t* row = states + i * kStateBytes;
        int result = row[OFF_RESULT], d = 0;
        load_position(P, row, t);
        __syncthreads();
        for (int ply = 0; ply < plies; ply++) {
            const bool act = live && result == 0;
            prepare_loaded(P, t);
            const ListInfo L = generate_legal(P, t);
            __syncthreads();
            if (act && t % kW == 0) {
                const int pick = (int)(((uint64_t)u[i * plies + ply] * (uint64_t)L.n) >> 32);
                int tp = MV_PASS, from = 0, to = 0, seg;
                if (L.total > 0) list_slot(P, L, pick, tp, from, to, seg);
                apply_mirrored(P, row, tp & 0xFF, tp >> 8, from, to);
                d++;
            }
            __syncthreads();
            result = P.result;
        }
        if (live && t % kW == 0) done[i] = d;
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

// The gated list of the immediate-win test against the whole list, per
// position: out[i] = {target cell, ub_total, whole-list total, gated hit,
// whole-list hit (the first 256 slots)}.  The target is the lone empty
// neighbour of the opponent's queen, else its first empty neighbour (a cell
// no move wins into: the gate still runs its bound), else -1.
void emu_gated_win(const uint8_t* states, int64_t B, int32_t* out) {
    run_group(64, (B + kPosPerWave - 1) / kPosPerWave, [&](int64_t w, int t) {
        int64_t i = w * kPosPerWave + t / kW;
        bool live = i < B;
        if (!live) i = B - 1;
        Pos& P = g_pos[t / kW];
        prepare(P, states + i * kStateBytes, t);
        const int me = P.turn & 1, opp = me ^ 1;
        int cell = lone_empty_cell(P, opp);
        if (cell < 0 && ((P.qplaced >> opp) & 1) && P.queen[opp] < kCells) {
            const int q = P.queen[opp];
            const uint32_t e = grid6(q) & ~nbr_bits_raw(P.occ, q);
            if (e) cell = step(q, __ffs(e) - 1);
        }
        const WinGate gate{cell, cell >= 0 ? (me ? 2 : 1) : 0};
        const ListInfo L = generate_legal(P, t, gate);
        const bool hg = wins_into(P, L, cell, t);
        __syncthreads();
        const ListInfo F = generate_legal(P, t);
        const bool hf = wins_into(P, F, cell, t);
        if (live && t % kW == 0) {
            int32_t* o = out + 5 * i;
            o[0] = cell;
            o[1] = L.ub_total;
            o[2] = F.total;
            o[3] = hg ? 1 : 0;
            o[4] = hf ? 1 : 0;
        }
    });
}

// The ant search's lifted-exit lookup against exits_lifted: every occupied
// cell c as the origin, every cell x of the grid; returns the mismatches.
int64_t emu_ring_exits_mismatches(const uint8_t* states, int64_t B) {
    std::atomic<int64_t> bad{0};
    run_group(64, (B + kPosPerWave - 1) / kPosPerWave, [&](int64_t w, int t) {
        int64_t i = w * kPosPerWave + t / kW;
        if (i >= B) i = B - 1;
        Pos& P = g_pos[t / kW];
        prepare(P, states + i * kStateBytes, t);
        for (int c = 0; c < kCells; c++) {
            if (!pb_get(P.occ, c)) continue;
            const Lift lf = lift_of(P, c);
            const RingLift rl = ring_lift(P, c);
            for (int x = t % kW; x < kCells; x += kW)
                if (exits_ring(P, x, rl) != exits_lifted(P, x, lf)) bad++;
        }
        __syncthreads();
    });
    return bad.load();
}

// div_exact against host IEEE division: the number of integers x in [lo, hi)
// where div_exact(x, d, rd) differs from x / d
int64_t emu_div_exact_mismatches(int64_t lo, int64_t hi, float d, float rd) {
    int64_t bad = 0;
    for (int64_t x = lo; x < hi; x++) {
        const volatile float want = (float)x / d;
        if (div_exact((float)x, d, rd) != want) bad++;
    }
    return bad;
}

// the same for the distance mean (s / n) / 10 of features_finish, n in 1..3, s in [0, smax)
int64_t emu_div_mean_mismatches(int64_t smax) {
    int64_t bad = 0;
    for (int n = 1; n <= 3; n++) {
        const float rn = n == 3 ? 1.f / 3.f : n == 2 ? 0.5f : 1.f;
        for (int64_t s = 0; s < smax; s++) {
            const volatile float m = (float)s / (float)n;
            const volatile float want = m / 10.0f;
            if (div_exact(div_exact((float)s, (float)n, rn), 10.0f, 0.1f) != want) bad++;
        }
    }
    return bad;
}

// has_immediate_surround_win_for_current_player as the probe runs it (immediate_win)
void emu_immediate_win(const uint8_t* states, int64_t B, uint8_t* out) {
    run_group(64, (B + kPosPerWave - 1) / kPosPerWave, [&](int64_t w, int t) {
        int64_t i = w * kPosPerWave + t / kW;
        bool live = i < B;
        if (!live) i = B - 1;
        prepare(g_pos[t / kW], states + i * kStateBytes, t);
        const bool win = immediate_win(g_pos[t / kW], t);
        if (live && t % kW == 0) out[i] = win ? 1 : 0;
    });
}

// root_tactical_probe_batch: the group programs of hive_probe.hpp in the
// order and with the bookkeeping of hive_probe.hip's launches.  cap: entries
// of the grandchild list (<= 0: B * 256, as the library sizes it; a small
// cap sends surviving candidates to the part programs).  Returns the number
// of candidates the part programs tested.
int64_t emu_root_probe(const uint8_t* states, const uint8_t* legal, const int32_t* nl, const float* pr, int64_t B, int f1,
                    int f2, int f3, int64_t* win, uint8_t* allowed, uint8_t* forced, int64_t cap) {
    if (cap <= 0) cap = B * 256;
    std::vector<RootProbe> R(B);
    run_group(64, (B + kPosPerWave - 1) / kPosPerWave, [&](int64_t w, int t) {
        int64_t i = w * kPosPerWave + t / kW;
        bool live = i < B;
        if (!live) i = B - 1;
        RootProbe rp = probe_root(g_pos[t / kW], states + i * kStateBytes, legal + i * 1536, nl[i], pr + i * 256,
                                  f1 != 0, f2 != 0, f3 != 0, t);
        if (live && t % kW == 0) R[i] = rp;
    });
    std::vector<int> js, jw;
    for (int64_t r = 0; r < B; r++) {
        for (int i = 0; i < 256; i++) allowed[r * 256 + i] = i < R[r].n;
        win[r] = R[r].win >= 0 ? R[r].win : ((R[r].gate & kProbeWin2) ? (1 << 20) : -1);
        if (R[r].gate & kProbeScreen)
            for (int i = 0; i < R[r].n; i++) js.push_back((int)(r * 256 + i));
        if (R[r].gate & kProbeWin2)
            for (int k = 0; k < 8; k++)
                for (uint32_t m = R[r].cand[k]; m; m &= m - 1) jw.push_back((int)(r * 256 + 32 * k + __builtin_ctz(m)));
    }
    int64_t ns = (int64_t)js.size(), nw = (int64_t)jw.size();
    if (ns)
        run_group(64, (ns + 1) / 2, [&](int64_t p, int t) {
            int64_t j = 2 * p + t / kW;
            bool live = j < ns;
            int job = js[live ? j : 2 * p];
            int64_t r = job / 256, i = job % 256;
            bool bad = probe_screen(g_pos[t / kW], states + r * kStateBytes, legal + (r * 256 + i) * 6, t);
            if (live && t % kW == 0) allowed[job] = bad ? 0 : 1;
        });
    std::vector<int> fail(nw, 0), over;
    std::vector<int32_t> gc(2 * cap, 0);
    unsigned long long reserved = 0;
    std::mutex over_mu;
    if (nw)
        run_group(64, (nw + 1) / 2, [&](int64_t p, int t) {
            int64_t j = 2 * p + t / kW;
            bool live = j < nw;
            if (!live) j = 2 * p;
            int job = jw[j];
            int64_t r = job / 256, i = job % 256;
            // independent of the screen (one launch in the library): every candidate
            int res = probe_drop_list(g_pos[t / kW], states + r * kStateBytes, legal + (r * 256 + i) * 6, live,
                                      (int32_t)j, &reserved, gc.data(), cap, t);
            if (live && t % kW == 0) {
                if (res == kDropped) __atomic_store_n(&fail[j], 1, __ATOMIC_SEQ_CST);
                else if (res == kOverflow) { std::lock_guard<std::mutex> g(over_mu); over.push_back((int)j); }
            }
        });
    const int64_t ng = (int64_t)reserved < cap ? (int64_t)reserved : cap;
    if (ng)
        run_group(64, (ng + 1) / 2, [&](int64_t p, int t) {
            int64_t g = 2 * p + t / kW;
            bool live = g < ng;
            if (!live) g = 2 * p;
            const int32_t j = gc[2 * g];
            int job = jw[j >= 0 ? j : 0];
            const bool active = live && j >= 0 && allowed[job] && __atomic_load_n(&fail[j], __ATOMIC_SEQ_CST) == 0;
            if (!hw_wave_any(active)) return;
            int64_t r = job / 256, i = job % 256;
            bool won = probe_grand(g_pos[t / kW], states + r * kStateBytes, legal + (r * 256 + i) * 6,
                                   (uint32_t)gc[2 * g + 1], t);
            if (active && !won && t % kW == 0) __atomic_store_n(&fail[j], 1, __ATOMIC_SEQ_CST);
        });
    const int64_t items = (int64_t)over.size() * kWin2Parts;
    if (items)
        run_group(64, (items + 1) / 2, [&](int64_t p, int t) {
            int64_t q = 2 * p + t / kW;
            bool live = q < items;
            if (!live) q = 2 * p;
            int64_t j = over[q / kWin2Parts];
            int job = jw[j];
            int64_t r = job / 256, i = job % 256;
            bool active = live && allowed[job];
            bool ok = probe_win2(g_pos[t / kW], g_rep[t / kW], states + r * kStateBytes, legal + (r * 256 + i) * 6,
                                 active, (int)(q % kWin2Parts), t);
            if (active && !ok && t % kW == 0) __atomic_store_n(&fail[j], 1, __ATOMIC_SEQ_CST);
        });
    for (int64_t j = 0; j < nw; j++) {
        int64_t r = jw[j] / 256, i = jw[j] % 256;
        if (allowed[jw[j]] && !fail[j] && i < win[r]) win[r] = i;
    }
    for (int64_t r = 0; r < B; r++) {
        if (win[r] == (1 << 20)) win[r] = -1;
        uint8_t f = 0;
        if (R[r].gate & kProbeScreen) {
            bool any = false;
            for (int i = 0; i < R[r].n; i++) any |= allowed[r * 256 + i] != 0;
            f = any ? 0 : 1;
        }
        forced[r] = f;
    }
    return (int64_t)over.size();
}
}
