// ref_capi.cpp -- C-ABI shim over the reference's own CPU build of its engine.
//
// TEST INFRASTRUCTURE ONLY.  It compiles the reference's
// hive_gpu/csrc/cpu_native.cpp exactly where it lies under /root/reference
// (that file already turns the .cuh headers into host C++), and exports
// plain C entry points so tests/golden/make_golden.py can write golden
// vectors and so the oracle can be cross-checked against the reference
// itself.  The built library goes to oracle/_ref/ (git-ignored) and is
// never part of the product.  No reference source is copied into this
// repository.
#include <cstring>
#include <thread>
#include <vector>

#include "cpu_native.cpp"  // resolved with -I<reference>/hive_gpu/csrc

using hive_gpu::GPUMove;
using hive_gpu::HiveState;

namespace {

HiveState load(const uint8_t* raw) {
    HiveState s;
    std::memcpy(&s, raw, sizeof(HiveState));
    return s;
}

template <typename F>
void split(int64_t n, int threads, F&& body) {
    if (threads < 1) threads = 1;
    if (threads == 1) {
        for (int64_t i = 0; i < n; ++i) body(i);
        return;
    }
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) {
        int64_t lo = n * t / threads, hi = n * (t + 1) / threads;
        pool.emplace_back([lo, hi, &body] {
            for (int64_t i = lo; i < hi; ++i) body(i);
        });
    }
    for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

int ref_state_bytes() { return (int)sizeof(HiveState); }

void ref_init() { hive_gpu::init_cpu_tables_once(); }

void ref_init_state(uint8_t* out, int mask) {
    hive_gpu::init_cpu_tables_once();
    HiveState s;
    std::memset(&s, 0, sizeof(s));
    hive_gpu::init_state(s, (uint8_t)mask);
    std::memcpy(out, &s, sizeof(s));
}

void ref_apply_move(uint8_t* raw, const uint8_t* mv6) {
    hive_gpu::init_cpu_tables_once();
    HiveState s = load(raw);
    GPUMove m;
    std::memcpy(&m, mv6, sizeof(m));
    hive_gpu::apply_move(s, m);
    std::memcpy(raw, &s, sizeof(s));
}

int ref_legal_moves(const uint8_t* raw, uint8_t* out) {
    hive_gpu::init_cpu_tables_once();
    HiveState s = load(raw);
    GPUMove mv[hive_gpu::MAX_LEGAL_MOVES];
    std::memset(mv, 0, sizeof(mv));
    int n = hive_gpu::generate_legal_moves(s, mv);
    std::memcpy(out, mv, sizeof(mv));
    return n;
}

int ref_fnn_feature_moves(const uint8_t* raw, uint8_t* out) {
    hive_gpu::init_cpu_tables_once();
    HiveState s = load(raw);
    GPUMove mv[hive_gpu::MAX_LEGAL_MOVES + 16];
    std::memset(mv, 0, sizeof(mv));
    int n = hive_gpu::generate_fnn_feature_moves(s, mv);
    std::memcpy(out, mv, sizeof(GPUMove) * hive_gpu::MAX_LEGAL_MOVES);
    return n;
}

void ref_fnn_features(const uint8_t* raw, const uint8_t* moves, int n, float* f) {
    hive_gpu::init_cpu_tables_once();
    HiveState s = load(raw);
    GPUMove mv[hive_gpu::MAX_LEGAL_MOVES];
    std::memset(mv, 0, sizeof(mv));
    std::memcpy(mv, moves, sizeof(GPUMove) * (size_t)n);
    hive_gpu::extract_fnn_features_device(s, mv, n, f);
}

void ref_articulation(const uint8_t* raw, uint64_t* out9) {
    hive_gpu::init_cpu_tables_once();
    HiveState s = load(raw);
    hive_gpu::Bitboard ap = hive_gpu::find_articulation_points(s);
    std::memcpy(out9, ap.w, sizeof(ap.w));
}

int ref_queen_escape(const uint8_t* raw) {
    hive_gpu::init_cpu_tables_once();
    HiveState s = load(raw);
    return hive_gpu::has_queen_escape_move(s) ? 1 : 0;
}

// legal moves + features per position, positions split statically over threads
void ref_batch_legal_features(const uint8_t* states, int64_t B, uint8_t* moves_out,
                              int32_t* n_out, float* feat_out, int threads) {
    hive_gpu::init_cpu_tables_once();
    split(B, threads, [&](int64_t i) {
        HiveState s = load(states + i * sizeof(HiveState));
        GPUMove mv[hive_gpu::MAX_LEGAL_MOVES];
        std::memset(mv, 0, sizeof(mv));
        int n = hive_gpu::generate_legal_moves(s, mv);
        if (moves_out) std::memcpy(moves_out + i * sizeof(mv), mv, sizeof(mv));
        if (n_out) n_out[i] = n;
        float f[hive_gpu::FNN_FEAT_DIM];
        hive_gpu::extract_fnn_features_device(s, mv, n, f);
        if (feat_out) std::memcpy(feat_out + i * hive_gpu::FNN_FEAT_DIM, f, sizeof(f));
    });
}

// successor features: apply move, then compact (full_list=0, the GPU
// orchestrator semantics of game_logic.cu:182-229) or full (full_list=1,
// cpu_native.cpp:130-174) legal list, then the 122 features.
void ref_batch_successor_features(const uint8_t* states, const uint8_t* legal,
                                  const int64_t* root, const int64_t* idx, int64_t N,
                                  float* feat_out, int full_list, int threads) {
    hive_gpu::init_cpu_tables_once();
    split(N, threads, [&](int64_t i) {
        HiveState child = load(states + root[i] * sizeof(HiveState));
        GPUMove m;
        std::memcpy(&m, legal + (root[i] * hive_gpu::MAX_LEGAL_MOVES + idx[i]) * sizeof(GPUMove),
                    sizeof(m));
        hive_gpu::apply_move(child, m);
        GPUMove mv[hive_gpu::MAX_LEGAL_MOVES + 16];
        int n = full_list ? hive_gpu::generate_legal_moves(child, mv)
                          : hive_gpu::generate_fnn_feature_moves(child, mv);
        hive_gpu::extract_fnn_features_device(child, mv, n, feat_out + i * hive_gpu::FNN_FEAT_DIM);
    });
}

// root_tactical_probe_kernel (game_logic.cu:290-397) for one root, composed
// from the reference's own primitives (apply_move, generate_legal_moves,
// has_immediate_surround_win_for_current_player,
// generate_non_decreasing_surround_replies, queen_surround_count_for_color_device).
// game_logic.cu is CUDA-only, so its loop is restated here around them.
void ref_root_tactical_probe(const uint8_t* raw, const uint8_t* moves, int nlegal, const float* priors, int win1,
                             int screen, int win2, int64_t* win_out, uint8_t* allowed, uint8_t* forced) {
    using namespace hive_gpu;
    init_cpu_tables_once();
    HiveState root = load(raw);
    std::vector<GPUMove> mv(MAX_LEGAL_MOVES);
    std::memcpy(mv.data(), moves, sizeof(GPUMove) * MAX_LEGAL_MOVES);
    *win_out = -1;
    *forced = 0;
    for (int i = 0; i < MAX_LEGAL_MOVES; ++i) allowed[i] = i < nlegal ? 1 : 0;
    if (nlegal <= 0 || root.result != IN_PROGRESS) return;
    Color me = current_player(root);
    Color opp = me == WHITE ? BLACK : WHITE;
    int opp_s = queen_surround_count_for_color_device(root, opp);
    int own_s = queen_surround_count_for_color_device(root, me);
    auto won = [&](const HiveState& s) {
        return (me == WHITE && s.result == WHITE_WINS) || (me == BLACK && s.result == BLACK_WINS);
    };
    if (win1 && opp_s == 5) {
        int best = -1;
        float bp = -1e30f;
        for (int i = 0; i < nlegal; ++i) {
            HiveState c = root;
            apply_move(c, mv[i]);
            if (won(c) && (best < 0 || priors[i] > bp)) {
                best = i;
                bp = priors[i];
            }
        }
        if (best >= 0) {
            *win_out = best;
            return;
        }
    }
    if (screen && own_s == 5) {
        bool any_safe = false;
        for (int i = 0; i < nlegal; ++i) {
            HiveState c = root;
            apply_move(c, mv[i]);
            bool bad = has_immediate_surround_win_for_current_player(c);
            allowed[i] = bad ? 0 : 1;
            any_safe |= !bad;
        }
        if (!any_safe) {
            *forced = 1;
            return;
        }
    }
    if (!win2 || !(opp_s == 4 || opp_s == 5)) return;
    std::vector<GPUMove> rep(MAX_LEGAL_MOVES);
    for (int i = 0; i < nlegal; ++i) {
        if (!allowed[i]) continue;
        HiveState c = root;
        apply_move(c, mv[i]);
        int cs = queen_surround_count_for_color_device(c, opp);
        if (opp_s == 4 && cs <= opp_s) continue;
        if (opp_s == 5 && cs < opp_s) continue;
        bool monotone = true;
        int nr = generate_non_decreasing_surround_replies(c, opp, cs, rep.data(), monotone);
        if (!monotone) continue;
        bool ok = true;
        for (int r = 0; r < nr && ok; ++r) {
            HiveState g = c;
            apply_move(g, rep[r]);
            if (!won(g) && !has_immediate_surround_win_for_current_player(g)) ok = false;
        }
        if (ok) {
            *win_out = i;
            return;
        }
    }
}

int ref_immediate_win(const uint8_t* raw) {
    hive_gpu::init_cpu_tables_once();
    HiveState s = load(raw);
    return hive_gpu::has_immediate_surround_win_for_current_player(s) ? 1 : 0;
}

}  // extern "C"
