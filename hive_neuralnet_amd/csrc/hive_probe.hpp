// hive_probe.hpp -- root tactical probe (root_tactical_probe_kernel,
// hive_gpu/csrc/game_logic.cu:290-397) as lane-group programs on the LDS
// board of hive_wave.hpp / hive_phases.hpp.
//
// The reference runs the whole probe of a root on one thread: an
// immediate-win scan, an opponent-immediate-win screen of every legal move
// (one full move generation per child) and a two-move forced-win search
// (one move generation per child and per reply).  Here each of those units
// is a 32-lane group program, so the move generations run lane-parallel and
// the (root, move) units of all roots run side by side (hive_probe.hip
// launches them):
//
//   probe_root    one root: surround counts, the immediate-win scan (lanes
//                 over the legal moves, each move's result decided from the
//                 occupancy change and queen cells it causes), the gates of
//                 the later stages and the two-move candidates;
//   probe_screen  one (root, move): the child, then
//                 has_immediate_surround_win_for_current_player on it;
//   probe_drop_list  one (root, candidate move): the child's replies and
//                 the non-decreasing-surround test over all of them (most
//                 candidates fail here, with no grandchild to test); a
//                 surviving candidate lists its grandchildren (the replies
//                 that do not already win for the root player);
//   probe_grand   one listed grandchild: the root player's immediate win;
//   probe_win2    one (surviving candidate whose grandchildren did not fit
//                 the list, part): the child's replies again, then the
//                 immediate-win test of every grandchild of the part that the
//                 reply does not already win.
//
// Every program reaches the same barriers in both groups of a wave: a group
// without work runs on the data it has and its caller writes nothing.
#pragma once

#include "hive_phases.hpp"

namespace hw {

enum { kProbeScreen = 1, kProbeWin2 = 2 };

// What a move changes that decides results and queen surround counts: the
// cell that becomes occupied, the cell that becomes empty (a lone piece
// leaving it) and the queen cells, as apply_on_board would leave them.
struct MoveEffect {
    int add, del;
    int q[2];
    uint32_t placed;
};

HW_INL MoveEffect move_effect(const Pos& P, int type, int pt, int from, int to) {
    MoveEffect e{-1, -1, {(int)P.queen[0], (int)P.queen[1]}, (uint32_t)P.qplaced};
    const int me = P.turn & 1;
    if (type == MV_PLACE) {
        if (to < kCells && pt >= PT_Q && pt <= PT_P && P.hgt(to) < 5) {
            e.add = to;
            if (pt == PT_Q) {
                e.q[me] = to;
                e.placed |= 1u << me;
            }
        }
    } else if (type == MV_MOVE) {
        if (from < kCells && to < kCells && P.hgt(from) > 0 && P.hgt(from) <= 5 && P.hgt(to) < 5) {
            int b = P.tp(from);
            if (P.hgt(from) == 1) e.del = from;
            e.add = to;
            if ((b & 15) == PT_Q) e.q[(b >> 4) & 1] = to;
        }
    }
    return e;
}

// queen_surround_count_for_color (game_logic.cu:257-263) after the move
HW_INL int surround_after(const Pos& P, const MoveEffect& e, int col) {
    if (!((e.placed >> col) & 1u)) return 0;
    int q = e.q[col];
    if (q < 0 || q >= kCells) return 0;
    uint32_t gm = grid6(q);
    uint32_t nb = nbr_bits_raw(P.occ, q) & gm;
    if (e.del >= 0) nb &= ~dir_bit_to(q, e.del, gm);
    if (e.add >= 0) nb |= dir_bit_to(q, e.add, gm);
    return __popc(nb);
}

HW_INL int surround_now(const Pos& P, int col) {
    MoveEffect e{-1, -1, {(int)P.queen[0], (int)P.queen[1]}, (uint32_t)P.qplaced};
    return surround_after(P, e, col);
}

// the result apply_move + check_game_over (hive_state.cuh:442-448,497-517) leave
HW_INL int result_after(const Pos& P, const MoveEffect& e) {
    bool w = surround_after(P, e, 0) == 6, b = surround_after(P, e, 1) == 6;
    if (w && b) return 3;
    if (w) return 2;
    if (b) return 1;
    return P.result;
}

// lone_empty_neighbor_of_queen (move_gen.cuh:833-851)
HW_INL int lone_empty_cell(const Pos& P, int target) {
    if (!((P.qplaced >> target) & 1)) return -1;
    int q = P.queen[target];
    if (q >= kCells) return -1;
    uint32_t gm = grid6(q);
    uint32_t nb = nbr_bits_raw(P.occ, q) & gm;
    if (__popc(nb) != 5) return -1;
    uint32_t e = gm & ~nb;
    if (__popc(e) != 1) return -1;
    return step(q, __ffs(e) - 1);
}

// hex distance between two cells of the 23x23 grid
__device__ __forceinline__ int hex_distance(int a, int b) {
    const int ra = row_of(a), rb = row_of(b);
    const int dq = (b - rb * kGrid) - (a - ra * kGrid), dr = rb - ra, ds = -(dq + dr);
    return max(max(abs(dq), abs(dr)), abs(ds));
}

// The pieces whose move to cell `stop` could win for the mover: the move's
// result (the opponent queen's sixth neighbour filled, the mover's own queen
// not surrounded with it) decides before any search, and the pieces that
// cannot get there in their own way are left out: one-step movers (queen,
// pillbug, beetle, a stacked mosquito) further than one cell, spiders and
// ladybugs further than three, and the sliding movers (queen, pillbug, ant,
// spider: their last step is a ground slide) when `stop` has no open side
// with the piece lifted -- a slide into a cell is a slide out of it, so its
// lifted slide exits (the exits of an empty cell) must not be empty.  Ant
// searches stop on reaching the cell.
struct WinGate {
    static constexpr bool kTargeted = true;
    int stop;
    int win;  // the mover's winning result (1 or 2); 0: run nothing
    HW_INL bool run(const Pos& P, int c, int t) const {
        if (stop < 0 || win == 0) return false;
        const int d = hex_distance(c, stop);
        if ((t == PT_Q || t == PT_P || t == PT_B || (t == PT_M && P.hgt(c) > 1)) && d != 1) return false;
        if ((t == PT_S || t == PT_L) && d > 3) return false;
        if ((t == PT_Q || t == PT_P || t == PT_A || t == PT_S) && exits_lifted(P, stop, lift_of(P, c)) == 0)
            return false;
        return result_after(P, move_effect(P, MV_MOVE, t, c, stop)) == win;
    }
};

// Moves of the (possibly gated) list L to `cell` that win for the mover: any
// slot before the cut; uniform within the group.
HW_INL bool wins_into(const Pos& P, const ListInfo& L, int cell, int lane) {
    const int me = P.turn & 1;
    bool hit = false;
    if (cell >= 0 && L.total > 0) {
        for (int i = gl(lane); i < L.n; i += kW) {
            int tp, from, to, seg;
            list_slot(P, L, i, tp, from, to, seg);
            if (to != cell) continue;
            MoveEffect e = move_effect(P, tp & 0xFF, tp >> 8, from, to);
            if (result_after(P, e) == (me ? 2 : 1)) hit = true;
        }
    }
    return grp_ballot(hit, lane) != 0;
}

// has_immediate_surround_win_for_current_player (move_gen.cuh:853-874) on a
// prepared board: some legal move to the lone empty neighbour of the
// opponent's queen wins, among the first 256 of the list.  Uniform within
// the group.  First a gated list (WinGate): only the pieces whose move to the
// cell would win are searched, the ant searches stop on the cell.  A gated
// list without such a move decides (no piece of the whole list has one); a
// gated list with one decides when the whole list is known to fit in 256
// slots (ub_total), else the full list is generated and scanned as the
// reference does.
template <bool kGated = true>
HW_INL bool immediate_win(Pos& P, int lane) {
    const int me = P.turn & 1;
    const int cell = lone_empty_cell(P, me ^ 1);
    const bool any = hw_wave_any(cell >= 0);
    if (!any) return false;  // neither group needs a list
    if (!kGated) return wins_into(P, generate_legal(P, lane), cell, lane);
    const WinGate gate{cell, cell >= 0 ? (me ? 2 : 1) : 0};
    const ListInfo L = generate_legal(P, lane, gate);
    bool hit = wins_into(P, L, cell, lane);
    const bool sure = !hit || L.ub_total <= kMaxLegal;
    if (hw_wave_any(!sure)) {  // a winning move that could lie past the cut
        __syncthreads();
        const ListInfo F = generate_legal(P, lane);
        const bool full = wins_into(P, F, cell, lane);
        if (!sure) hit = full;
    }
    return hit;
}

struct RootProbe {
    int win;        // immediate win found (slot), else -1
    int gate;       // kProbeScreen | kProbeWin2: the later stages that run
    int n;          // legal moves considered (num_legal clamped to 256)
    int opp_s;      // the opponent's queen surround count
    uint32_t cand[8];  // two-move candidates: moves that raise (opp_s 4) / keep (opp_s 5) it
};

// probe_root: stages 1 and the gates of 2 and 3 of root_tactical_probe_kernel.
// M: the root's [256][6] legal list, n its count, pr its priors.
HW_INL RootProbe probe_root(Pos& P, const uint8_t* __restrict__ S, const uint8_t* __restrict__ M, int n,
                            const float* __restrict__ pr, bool win1, bool screen, bool win2, int lane) {
    const int l = gl(lane);
    load_position(P, S, lane);
    __syncthreads();
    RootProbe R{-1, 0, n < 0 ? 0 : (n > kMaxLegal ? kMaxLegal : n), 0, {0, 0, 0, 0, 0, 0, 0, 0}};
    const bool go = R.n > 0 && P.result == 0;
    const int me = P.turn & 1;
    const int opp_s = surround_now(P, me ^ 1), own_s = surround_now(P, me);
    R.opp_s = opp_s;
    if (!go) return R;
    if (win1 && opp_s == 5) {
        uint32_t wins[8];
        for (int k = 0; k < 8; k++) {
            int i = 32 * k + l;
            bool w = false;
            if (i < R.n) {
                const uint8_t* m = M + 6 * i;
                MoveEffect e = move_effect(P, m[0], m[1], m[2] | (m[3] << 8), m[4] | (m[5] << 8));
                w = result_after(P, e) == (me ? 2 : 1);
            }
            wins[k] = grp_ballot(w, lane);
        }
        // first winning slot, replaced only by a strictly higher prior
        int best = -1;
        float bp = -1e30f;
        for (int k = 0; k < 8; k++) {
            uint32_t w = wins[k];
            while (w) {
                int i = 32 * k + __ffs(w) - 1;
                w &= w - 1;
                float p = pr[i];
                if (best < 0 || p > bp) {
                    best = i;
                    bp = p;
                }
            }
        }
        if (best >= 0) {
            R.win = best;
            return R;
        }
    }
    if (screen && own_s == 5) R.gate |= kProbeScreen;
    if (win2 && (opp_s == 4 || opp_s == 5)) {
        R.gate |= kProbeWin2;
        for (int k = 0; k < 8; k++) {
            int i = 32 * k + l;
            bool c = false;
            if (i < R.n) {
                const uint8_t* m = M + 6 * i;
                MoveEffect e = move_effect(P, m[0], m[1], m[2] | (m[3] << 8), m[4] | (m[5] << 8));
                int cs = surround_after(P, e, me ^ 1);
                c = opp_s == 4 ? cs > opp_s : cs >= opp_s;
            }
            R.cand[k] = grp_ballot(c, lane);
        }
    }
    return R;
}

// probe_screen: does the opponent win at once after the root move m?
HW_INL bool probe_screen(Pos& P, const uint8_t* __restrict__ S, const uint8_t* __restrict__ m, int lane) {
    load_position(P, S, lane);
    __syncthreads();
    if (gl(lane) == 0) apply_on_board(P, S, m[0], m[1], m[2] | (m[3] << 8), m[4] | (m[5] << 8));
    __syncthreads();
    prepare_loaded(P, lane);
    return immediate_win<false>(P, lane);
}

// the child's replies, kept while grandchildren are evaluated on the board
struct Replies {
    uint8_t mv[kMaxLegal][6];
    uint32_t need[8];  // replies whose grandchild must be tested for an immediate win
    int n;
};

// A candidate's child board, its replies' list and the opponent queen's
// surround on the child (the replies are the opponent's moves).
struct ChildList {
    ListInfo L;
    int opp, cs;
};
HW_INL ChildList child_replies(Pos& P, const uint8_t* __restrict__ S, const uint8_t* __restrict__ m, int lane,
                               BaseRegs* child = nullptr) {
    load_position(P, S, lane);
    __syncthreads();
    if (gl(lane) == 0) apply_on_board(P, S, m[0], m[1], m[2] | (m[3] << 8), m[4] | (m[5] << 8));
    __syncthreads();
    if (child) save_base(P, *child, lane);
    prepare_loaded(P, lane);
    ChildList C;
    C.opp = P.turn & 1;
    C.cs = surround_now(P, C.opp);
    C.L = generate_legal(P, lane);
    return C;
}

// slot i of the replies' list (a lone PASS when the list is empty)
HW_INL MoveEffect reply_effect(const Pos& P, const ListInfo& L, int i) {
    int tp = MV_PASS, from = 0, to = 0, seg;
    if (L.total > 0) list_slot(P, L, i, tp, from, to, seg);
    return move_effect(P, tp & 0xFF, tp >> 8, from, to);
}

// A reply packed for the grandchild list: move type (2 bits), piece type
// (4), from (10), to (10).  Listed moves have both cells below kCells
// (placements and PASS carry from = 0), so the packing is lossless.
static_assert(kCells <= 1024 && MV_PASS < 4, "reply fields in 26 bits");
__device__ __forceinline__ uint32_t pack_reply(int tp, int from, int to) {
    return ((uint32_t)tp & 3u) | (((uint32_t)tp >> 8) & 15u) << 2 | (uint32_t)from << 6 | (uint32_t)to << 16;
}

// probe_drop: after root move m, does some reply lower the opponent queen's
// surround below its level after m (generate_non_decreasing_surround_replies,
// move_gen.cuh:876-898, finds a reply it leaves out)?  Such a candidate is no
// forced win whatever the grandchildren hold: kDropped.  Otherwise every
// reply that does not already win for the root player leaves a grandchild
// to test; an `active` group reserves that many entries of the grandchild
// list (gc: pairs of int32, the candidate's index `cand` and the packed
// reply; *count counts reservations in 64 bits, cap entries fit) and writes them:
// kListed.  A reservation that does not fit writes the sentinel -1 into the
// entries of its range below cap and returns kOverflow (the caller tests
// that candidate's grandchildren by the part programs).  A child that is a
// finished game (m won) has no replies and lists nothing.  Uniform within
// the group.
enum { kDropped = 0, kListed = 1, kOverflow = 2 };
HW_INL int probe_drop_list(Pos& P, const uint8_t* __restrict__ S, const uint8_t* __restrict__ m, bool active,
                           int32_t cand, unsigned long long* __restrict__ count, int32_t* __restrict__ gc,
                           int64_t cap, int lane) {
    const int l = gl(lane);
    const ChildList C = child_replies(P, S, m, lane);
    const int win = (C.opp ^ 1) ? 2 : 1;
    bool drop = false;
    uint32_t need[8];
    int n_need = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = 32 * k + l;
        bool nd = false;
        if (i < C.L.n) {
            const MoveEffect e = reply_effect(P, C.L, i);
            if (surround_after(P, e, C.opp) < C.cs) drop = true;
            nd = result_after(P, e) != win;
        }
        need[k] = grp_ballot(nd, lane);
        n_need += __popc(need[k]);
    }
    if (grp_ballot(drop, lane) != 0) return kDropped;
    const int want = active ? n_need : 0;
    int64_t base = 0;
    if (l == 0 && want > 0) base = (int64_t)atomicAdd(count, (unsigned long long)want);
    base = grp_shfl(base, 0, lane);
    const bool fits = base + want <= cap;
    int rank = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        if (want > 0 && ((need[k] >> l) & 1u)) {
            const int64_t e = base + rank + __popc(need[k] & ((1u << l) - 1u));
            if (fits) {
                int tp = MV_PASS, from = 0, to = 0, seg;
                if (C.L.total > 0) list_slot(P, C.L, 32 * k + l, tp, from, to, seg);
                gc[2 * e] = cand;
                gc[2 * e + 1] = (int32_t)pack_reply(tp, from, to);
            } else if (e < cap) {
                gc[2 * e] = -1;
            }
        }
        rank += __popc(need[k]);
    }
    return fits ? kListed : kOverflow;
}

// probe_grand: one grandchild of the two-move search -- the root row S,
// root move m, then the packed reply -- does the root player win at once?
// (The piece a move reveals is read from S: the levels under a top are
// unchanged by two moves, since a reply can only lift what m put on top.)
HW_INL bool probe_grand(Pos& P, const uint8_t* __restrict__ S, const uint8_t* __restrict__ m, uint32_t reply,
                        int lane) {
    load_position(P, S, lane);
    __syncthreads();
    if (gl(lane) == 0) {
        apply_on_board(P, S, m[0], m[1], m[2] | (m[3] << 8), m[4] | (m[5] << 8));
        apply_on_board(P, S, (int)(reply & 3u), (int)((reply >> 2) & 15u), (int)((reply >> 6) & 1023u),
                       (int)((reply >> 16) & 1023u));
    }
    __syncthreads();
    prepare_loaded(P, lane);
    return immediate_win(P, lane);
}

// The grandchildren of one candidate are split over kWin2Parts programs (part
// p tests the replies whose slot is p modulo kWin2Parts), so a candidate with
// many replies is not one long serial walk; the candidate passes when no part
// fails.
constexpr int kWin2Parts = 64;
static_assert(kWin2Parts > 0 && kWin2Parts <= kMaxLegal && (kWin2Parts & (kWin2Parts - 1)) == 0,
              "parts: a power of two, at most one slot each");

// probe_win2, for a candidate that passed probe_drop_list (no reply lowers the
// opponent queen's surround): does every reply of this part leave a position
// the root player has already won or wins at once?  `active` false: the
// group follows the other group of its wave and its result is meaningless.
HW_INL bool probe_win2(Pos& P, Replies& Rp, const uint8_t* __restrict__ S, const uint8_t* __restrict__ m,
                       bool active, int part, int lane) {
    const int l = gl(lane);
    // the child's base fields, put back before each reply instead of
    // reloading the root and applying m again
    BaseRegs child;
    const ChildList C = child_replies(P, S, m, lane, &child);
    const ListInfo& L = C.L;
    const int me = C.opp ^ 1;
    // the replies of this part that do not already win for the root player,
    // decoded (a lone PASS when the list is empty) and kept by slot
    for (int k = 0; k < 8; k++) {
        const int i = 32 * k + l;
        bool need = false;
        if (i < L.n && (i & (kWin2Parts - 1)) == part) {
            int tp = MV_PASS, from = 0, to = 0, seg;
            if (L.total > 0) list_slot(P, L, i, tp, from, to, seg);
            need = result_after(P, move_effect(P, tp & 0xFF, tp >> 8, from, to)) != (me ? 2 : 1);
            if (need) {
                Rp.mv[i][0] = (uint8_t)(tp & 0xFF);
                Rp.mv[i][1] = (uint8_t)(tp >> 8);
                Rp.mv[i][2] = (uint8_t)from;
                Rp.mv[i][3] = (uint8_t)(from >> 8);
                Rp.mv[i][4] = (uint8_t)to;
                Rp.mv[i][5] = (uint8_t)(to >> 8);
            }
        }
        const uint32_t nw = grp_ballot(need, lane);
        if (l == 0) Rp.need[k] = nw;
    }
    if (l == 0) Rp.n = L.n;
    bool ok = active;
    __syncthreads();
    // every remaining grandchild: the root player wins at once (any order;
    // the first failure decides)
    int k = 0;
    uint32_t w = Rp.need[0];
    for (;;) {
        while (w == 0 && k < 7) w = Rp.need[++k];
        const bool more = ok && w != 0;
        if (!hw_wave_any(more)) break;
        int r = more ? 32 * k + __ffs(w) - 1 : -1;
        if (more) w &= w - 1;
        restore_base(P, child, lane);
        __syncthreads();
        if (l == 0 && r >= 0)
            apply_on_board(P, S, Rp.mv[r][0], Rp.mv[r][1], Rp.mv[r][2] | (Rp.mv[r][3] << 8),
                           Rp.mv[r][4] | (Rp.mv[r][5] << 8));
        __syncthreads();
        prepare_loaded(P, lane);
        bool won = immediate_win(P, lane);
        if (more && !won) ok = false;
        __syncthreads();
    }
    return ok;
}

}  // namespace hw
