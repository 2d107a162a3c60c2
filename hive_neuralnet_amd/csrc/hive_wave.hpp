// hive_wave.hpp -- wave-cooperative Hive rules engine for CDNA4 (gfx950).
//
// A group of kW = 32 lanes owns one position; a 64-lane wavefront works on
// two positions side by side (lanes 0-31 and 32-63), so the sequential
// parts of a position (searches of single pieces, floods, per-word loops)
// are paid once per two positions.  The board lives in LDS as
//   * padded 32-bit-word bitboards (occupied / white top / black top /
//     articulation / pinned / placement): board word w sits at index w+1,
//     indices 0 and 19 are zero pads so that any cell's 47-bit neighbour
//     window (cells c-23 .. c+23) is three aligned word reads;
//   * per-cell height and top-piece bytes, and per-cell 6-bit direction
//     masks of occupied neighbours (nb) and of ground-slide exits (sm),
//     built once per board so that the generators' inner loops read one
//     byte instead of rebuilding a neighbour window.
// Work is spread over lanes by what is parallel in each phase: board words
// (placements, list building), occupied cells (articulation points,
// features), movable pieces (destination generation), legal-list slots
// (assembly, action indices).
//
// Semantics follow the reference engine (chrismejias/hive_neuralnet,
// hive_gpu/csrc/*.cuh); each routine cites what it reproduces.  Outputs are
// bit-exact with it for states produced by init/apply (the only states the
// reference API produces): the occupancy bitboards are taken as consistent
// with the height array, as apply keeps them.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "hw_target.hpp"

namespace hw {

constexpr int kCells = 529;
constexpr int kGrid = 23;
constexpr int kHalf = 11;
constexpr int kStateBytes = 3424;
constexpr int kMaxLegal = 256;
constexpr int kFeat = 122;
constexpr int kPW = 20;  // padded words per bitboard
constexpr int kMaxPieces = 16;
// Destination pool entries for one side's pieces at type_capacity() each:
// 3 ants x 60 + mosquito 96 + 2 spiders x 32 + ladybug 32 + 8 others x 6.
// Capacities are bounds for states built by init/apply: a connected hive of
// n cells has at most 2n + 4 empty neighbour cells (each cell added next to
// the hive removes one and adds at most three), every ant destination is
// one of them with n <= 27 (the ant lifted), so an ant has <= 58; a
// mosquito's union (<= 58 empty cells + 6 neighbours to climb on) plus the
// sub-list being merged (<= 32) fits in 96.
constexpr int kAntCap = 60;
// Ant searches: one lane per ant (gen_ant).  Built with HW_ANT_GROUP = T > 0,
// a lane makes at most T expansions and the lane group finishes the longer
// searches together (ant_searches): bit-exact, but slower on the measured
// workloads, so the default build keeps the lane searches.
#ifndef HW_ANT_GROUP
#define HW_ANT_GROUP 0
#endif
constexpr int kMosqRoom = 96;
constexpr int kPool = 3 * kAntCap + kMosqRoom + 2 * 32 + 32 + 8 * 6;
constexpr int kActors = 2;  // throw actors of one colour: its pillbug and its mosquito
// throws of one actor: targets are occupied and drops empty neighbours of
// the actor, so targets x drops <= 3 x 3
constexpr int kThrowCap = 9;
constexpr int kSets = 8;  // visited / dedup sets: 3 ants, 2 spiders, 1 ladybug, 1 mosquito (2)
constexpr int kPlist = 240;  // placement cells kept for emission (a board has <= 60)
constexpr int kSegs = 1 + kMaxPieces + kActors + 1;  // placements, pieces, actors, end
constexpr int kArtN = 28;  // vertices (occupied cells in cell order) the articulation test covers
constexpr int kW = 32;               // lanes per position
constexpr int kPosPerWave = 64 / kW;  // positions per wavefront

// state byte offsets (hive_gpu/csrc/hive_state.cuh:239-269)
constexpr int OFF_HEIGHT = 2645, OFF_OCC = 3176, OFF_WTOP = 3248, OFF_BTOP = 3320;
constexpr int OFF_QUEEN = 3392, OFF_HANDS = 3396, OFF_TURN = 3412, OFF_QPLACED = 3414;
constexpr int OFF_RESULT = 3415, OFF_STUN = 3416;

enum { PT_Q = 1, PT_A = 2, PT_G = 3, PT_S = 4, PT_B = 5, PT_M = 6, PT_L = 7, PT_P = 8 };
enum { MV_PLACE = 0, MV_MOVE = 1, MV_PASS = 2 };

// Direction d in E, NE, NW, W, SW, SE order (hex_grid.cuh:32-42).  The cell
// offset of direction d is OFS(d) - 23 where OFS packs 6-bit fields; OFS(d)
// is also d's bit position in the 47-bit window starting at cell c-23.
constexpr uint64_t kOfs = (24ull) | (1ull << 6) | (0ull << 12) | (22ull << 18) | (45ull << 24) | (46ull << 30);
__device__ __forceinline__ int win_ofs(int d) { return (int)((kOfs >> (6 * d)) & 63); }
__device__ __forceinline__ int step(int c, int d) { return c + win_ofs(d) - 23; }

// grid row of a cell: c / 23 for 0 <= c < 4096 (one multiply and a shift;
// (c * 2850) >> 16 equals c / 23 over that whole range)
__device__ __forceinline__ int row_of(int c) { return (int)(((uint32_t)c * 2850u) >> 16); }

// directions whose neighbour is on the 23x23 grid
__device__ __forceinline__ uint32_t grid6(int c) {
    int r = row_of(c), col = c - r * kGrid;
    uint32_t m = 0;
    if (col < 22) m |= 1u;
    if (col < 22 && r > 0) m |= 2u;
    if (r > 0) m |= 4u;
    if (col > 0) m |= 8u;
    if (col > 0 && r < 22) m |= 16u;
    if (r < 22) m |= 32u;
    return m;
}

__device__ __forceinline__ uint32_t rotl6(uint32_t n) { return ((n << 1) | (n >> 5)) & 63u; }
__device__ __forceinline__ uint32_t rotr6(uint32_t n) { return ((n >> 1) | (n << 5)) & 63u; }

__device__ __forceinline__ int pb_get(const uint32_t* pb, int c) { return (int)((pb[(c >> 5) + 1] >> (c & 31)) & 1u); }

// 64 board bits starting at bit lo (>= -32) of a padded bitboard
__device__ __forceinline__ uint64_t bit_window(const uint32_t* pb, int lo) {
    int wi = (lo >> 5) + 1;
    int sh = lo & 31;
    uint64_t w01 = (uint64_t)pb[wi] | ((uint64_t)pb[wi + 1] << 32);
    uint64_t win = w01 >> sh;
    if (sh) win |= (uint64_t)pb[wi + 2] << (64 - sh);
    return win;
}
// the six direction bits of a window that starts at cell c - 23
__device__ __forceinline__ uint32_t ring_bits(uint64_t win) {
    return (uint32_t)((win >> 24) & 1u) | (uint32_t)(((win >> 1) & 1u) << 1) |
           (uint32_t)((win & 1u) << 2) | (uint32_t)(((win >> 22) & 1u) << 3) |
           (uint32_t)(((win >> 45) & 1u) << 4) | (uint32_t)(((win >> 46) & 1u) << 5);
}
// 6-bit mask of directions d whose neighbour is on-grid and set in pb.
// Bits c-23 .. c+40 are gathered into one 64-bit window; direction d sits at
// window bit win_ofs(d).
__device__ __forceinline__ uint32_t nbr_bits_raw(const uint32_t* pb, int c) { return ring_bits(bit_window(pb, c - 23)); }
__device__ __forceinline__ uint32_t nbr_bits(const uint32_t* pb, int c) { return nbr_bits_raw(pb, c) & grid6(c); }

// 32 board bits starting at bit_off (>= -32) of a padded bitboard
__device__ __forceinline__ uint32_t word_field(const uint32_t* pb, int bit_off) {
    int wi = (bit_off >> 5) + 1;
    int sh = bit_off & 31;
    uint64_t v = (uint64_t)pb[wi] | ((uint64_t)pb[wi + 1] << 32);
    return (uint32_t)(v >> sh);
}

// window positions (cell offset + 23) of the six directions, as a bit set
constexpr uint64_t kRingWin = (1ull << 24) | (1ull << 1) | (1ull << 0) | (1ull << 22) | (1ull << 45) | (1ull << 46);

// direction bit of g as seen from c (0 when g is not c's on-grid neighbour)
__device__ __forceinline__ uint32_t dir_bit_to(int c, int g, uint32_t gm) {
    int w = g - c + 23;
    uint32_t b = (uint32_t)(w == 24) | ((uint32_t)(w == 1) << 1) | ((uint32_t)(w == 0) << 2) |
                 ((uint32_t)(w == 22) << 3) | ((uint32_t)(w == 45) << 4) | ((uint32_t)(w == 46) << 5);
    return b & gm;
}

struct alignas(16) Pos {
    // pin: articulation points whose stack is one piece high
    uint32_t occ[kPW], wt[kPW], bt[kPW], pin[kPW], plc[kPW];
    uint8_t cell[544];  // top piece byte (type | colour << 4) in bits 0-4, stack height in bits 5-7
    uint8_t sm[532];  // ground-slide exits of each board cell with nothing lifted
    uint16_t occ_pre[20];  // occupied cells in board words before word w
    uint16_t plc_pre[20];  // placement cells in board words before word w
    int16_t seg_base[32];  // legal-list segment starts (placements, pieces, actors, end); 32767 past the end
    uint16_t queen[2];
    uint16_t turn, stun;
    uint8_t hand[2][8];
    uint8_t qplaced, result, pad_[2];
    int n_occ;
    uint16_t occ_cells[32];
    uint8_t nbd[32];  // occupied on-grid neighbours (direction mask) of the occupied cells, by rank
    // move generation
    int n_pieces, n_actors, n_place, n_total;
    uint16_t piece_cell[kMaxPieces];
    uint8_t piece_type[kMaxPieces];
    uint16_t piece_off[kMaxPieces];
    uint8_t piece_cnt[kMaxPieces];
    int16_t piece_win[kMaxPieces];  // action-window index of each piece cell (emission)
    uint16_t actor_cell[kActors];
    uint16_t throw_cnt[kActors];
    uint16_t throw_from[kActors][kThrowCap];
    uint16_t throw_to[kActors][kThrowCap];
    uint8_t throw_pt[kActors][kThrowCap];
    // articulation: dense adjacency; generation: visited sets; emission and
    // features: the generated list's MOVE sources per (type, owner), by rank,
    // and the placement cells in ascending order (the first kPlist)
    union {
        uint32_t adj[32];
        uint32_t sets[kSets][17];
        struct {
            uint32_t from_d[16];
            uint16_t plist[kPlist];
        } e;
    } u1;
    // generation and emission: destinations; features (after emission): counters
    union {
        uint16_t pool[kPool];
        struct {
            int cnt[128];
            int dsum[16], dcnt[16];
            int ring[2], covered[2], capable[2];
            int n_cap;
            uint16_t cap_cells[8];
            uint8_t cap_col[8];
        } c;
    } u2;
    __device__ __forceinline__ int hgt(int c) const { return cell[c] >> 5; }
    __device__ __forceinline__ int tp(int c) const { return cell[c] & 31; }
    __device__ __forceinline__ void set_cell(int c, int h, int top) {
        cell[c] = (uint8_t)((h << 5) | (h ? (top & 31) : 0));
    }
};

static_assert(offsetof(Pos, hand) % 4 == 0, "hand rows are read as two dwords each");

// Bit p set when colour col holds pieces of type p + 1 in hand.  Four hand
// bytes at a time: bit 7 of (b & 0x7F) + 0x7F, or'ed with b, is set iff b is
// non-zero (no carry leaves a byte); the bits 7, 15, 23, 31 are gathered to
// bits 28..31 by one multiply (the partial products land on distinct bits).
__device__ __forceinline__ uint32_t hand_mask(const Pos& P, int col) {
    const uint32_t* h = reinterpret_cast<const uint32_t*>(P.hand[col]);
    auto nz4 = [](uint32_t x) {
        const uint32_t t = ((((x & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | x) & 0x80808080u) >> 7;
        return (t * 0x10204080u) >> 28;
    };
    return nz4(h[0]) | (nz4(h[1]) << 4);
}

// MOVE sources per (type, owner) and PLACE destinations of a caller-supplied
// list, as bitboards over all cells (the list may name any cell)
struct ListSets {
    uint32_t from_bb[16][18];
    uint32_t place_bb[18];
};

// ---------------------------------------------------------------- wave utils
// Inclusive prefix sum over the 64 lanes with DPP lane moves: shifts by 1,
// 2, 4, 8 within each 16-lane row, then the row totals carried by
// row_bcast:15 (into rows 1, 3) and row_bcast:31 (into rows 2, 3).
// Lanes a move has no source for add 0 (bound_ctrl), so do disabled rows.
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, true);  // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, true);  // row_bcast:31
    return x;
}

__device__ __forceinline__ int wave_excl_scan(int v, int lane) {
    (void)lane;
    return wave_incl_scan(v) - v;
}

__device__ __forceinline__ int wave_sum(int v) { return __builtin_amdgcn_readlane(wave_incl_scan(v), 63); }

// ---- lane-group (one position) versions; `lane` is the wavefront lane
__device__ __forceinline__ int gl(int lane) { return lane & (kW - 1); }

// inclusive prefix sum within each 32-lane group: row shifts, then the row
// total of rows 0 / 2 carried into rows 1 / 3 (row_bcast:15)
__device__ __forceinline__ int grp_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, true);  // row_bcast:15
    return x;
}
__device__ __forceinline__ int grp_excl_scan(int v) { return grp_incl_scan(v) - v; }
template <typename T>
__device__ __forceinline__ T grp_shfl(T v, int src, int lane) { return __shfl(v, (lane & ~(kW - 1)) | src, 64); }
__device__ __forceinline__ int grp_sum(int v, int lane) { return grp_shfl(grp_incl_scan(v), kW - 1, lane); }
__device__ __forceinline__ uint32_t grp_ballot(bool p, int lane) {
    return (uint32_t)(__ballot(p) >> (lane & ~(kW - 1)));
}
__device__ __forceinline__ uint32_t grp_or(uint32_t v) {
#pragma unroll
    for (int o = kW / 2; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
    return v;
}

// ---------------------------------------------------------------- state load
// Four cells' bytes (height in bits 5-7, clamped to 7; top piece in bits 0-4
// when the stack is non-empty) from their heights and level-0 bytes, four
// bytes at a time (no byte carries into its neighbour: every per-byte sum
// stays below 256); bit k of *stacked is set for byte k when its top is above
// level 0.  Cells past the board must come with height 0.
__device__ __forceinline__ uint32_t pack_cells4(uint32_t hts, uint32_t lv0, uint32_t& stacked) {
    const uint32_t big = ((((hts & 0xF8F8F8F8u) >> 3) + 0x1F1F1F1Fu) >> 5) & 0x01010101u;  // height >= 8
    const uint32_t h7 = (hts & 0x07070707u) | (big * 7u);                               // min(height, 7)
    const uint32_t nz = ((h7 + 0x7F7F7F7Fu) >> 7) & 0x01010101u;                        // height >= 1
    const uint32_t up = ((h7 + 0x7E7E7E7Eu) >> 7) & 0x01010101u;                        // height >= 2
    stacked = ((up * 0x00204081u) >> 21) & 15u;  // byte k's flag (bit 8k) lands on bit 21 + k
    return (h7 << 5) | (lv0 & 0x1F1F1F1Fu & (nz * 0xFFu));
}

// Heights, top bytes, bitboards and metadata of the state row S into P.
// Lane l of the group takes the 16-cell chunk l (cells 16l .. 16l + 15): its
// level-0 bytes (one 16-byte load) and its heights, which start at the odd
// offset 2645 (a 16-byte and a 4-byte load, realigned in registers); lanes
// 0-4 also take the four cells 512 + 4l .. 515 + 4l (cells 529-531 are past
// the board: their height bytes are masked off).  Every load of the position
// is issued before the first is used, so the whole row costs one memory
// round trip; the top byte of a stack (height > 1) is a second, rare,
// dependent load.
HW_INL void load_position(Pos& P, const uint8_t* __restrict__ S, int lane) {
    const int l = gl(lane);
    static_assert(kCells == 16 * kW + 17 && kW == 32, "32 chunks of 16 cells, then 17 cells in five words");
    const bool tail = l < 5;
    u32x4 lv_a = *reinterpret_cast<const u32x4*>(S + 16 * l);
    u32x4 ht_a = *reinterpret_cast<const u32x4*>(S + (OFF_HEIGHT - 1) + 16 * l);
    uint32_t ht_a4 = *reinterpret_cast<const uint32_t*>(S + (OFF_HEIGHT - 1) + 16 * l + 16);
    uint32_t lv_t = 0, ht_t0 = 0, ht_t1 = 0;
    if (tail) {
        lv_t = *reinterpret_cast<const uint32_t*>(S + 512 + 4 * l);
        ht_t0 = *reinterpret_cast<const uint32_t*>(S + (OFF_HEIGHT - 1) + 512 + 4 * l);
        ht_t1 = *reinterpret_cast<const uint32_t*>(S + (OFF_HEIGHT - 1) + 516 + 4 * l);
    }
    const uint32_t* W = reinterpret_cast<const uint32_t*>(S + OFF_OCC);  // 8-byte aligned
    uint32_t occ_w = 0, wt_w = 0, bt_w = 0;
    if (l < 18) {
        occ_w = W[l];
        wt_w = W[18 + l];
        bt_w = W[36 + l];
    }
    uint32_t m0 = 0, m1 = 0, m2 = 0, m3 = 0, m4 = 0, m5 = 0, m6 = 0;
    if (l == 24) {
        const uint32_t* M = reinterpret_cast<const uint32_t*>(S + OFF_QUEEN);
        m0 = M[0]; m1 = M[1]; m2 = M[2]; m3 = M[3]; m4 = M[4]; m5 = M[5]; m6 = M[6];
    }

    uint32_t* cell32 = reinterpret_cast<uint32_t*>(P.cell);
    uint32_t st_a = 0, st_t = 0;
    {
        u32x4 o;
        uint32_t s0, s1, s2, s3;
        o[0] = pack_cells4(__builtin_amdgcn_alignbyte(ht_a[1], ht_a[0], 1), lv_a[0], s0);
        o[1] = pack_cells4(__builtin_amdgcn_alignbyte(ht_a[2], ht_a[1], 1), lv_a[1], s1);
        o[2] = pack_cells4(__builtin_amdgcn_alignbyte(ht_a[3], ht_a[2], 1), lv_a[2], s2);
        o[3] = pack_cells4(__builtin_amdgcn_alignbyte(ht_a4, ht_a[3], 1), lv_a[3], s3);
        st_a = s0 | (s1 << 4) | (s2 << 8) | (s3 << 12);
        *reinterpret_cast<u32x4*>(cell32 + 4 * l) = o;
    }
    if (tail) {  // board word 128 + l; word 132 holds cell 528 only
        const uint32_t keep = l == 4 ? 0xFFu : 0xFFFFFFFFu;
        cell32[128 + l] = pack_cells4(__builtin_amdgcn_alignbyte(ht_t1, ht_t0, 1) & keep, lv_t, st_t);
    } else if (l < 8) {
        cell32[128 + l] = 0u;  // words 133-135: cells 532-543, past the board
    }
    // stacked tops: level min(h, 5) - 1 of the cell (h is the clamped height)
    uint32_t st = st_a | (st_t << 16);
    while (st) {
        int b = __ffs(st) - 1;
        st &= st - 1;
        int c = b < 16 ? 16 * l + b : 512 + 4 * l + (b - 16);
        int h = P.cell[c] >> 5;
        int t = S[((h > 5 ? 5 : h) - 1) * kCells + c];
        P.cell[c] = (uint8_t)((h << 5) | (t & 31));
    }

    if (l < 18) {
        P.occ[l + 1] = occ_w;
        P.wt[l + 1] = wt_w;
        P.bt[l + 1] = bt_w;
    } else if (l < 24) {
        int k = l - 18;  // zero the pads: k = 0 -> index 0, k = 1 -> index 19
        uint32_t* dst = k < 2 ? P.occ : k < 4 ? P.wt : P.bt;
        dst[(k & 1) ? 19 : 0] = 0;
    } else if (l == 24) {
        P.queen[0] = (uint16_t)m0;
        P.queen[1] = (uint16_t)(m0 >> 16);
        uint32_t* hand32 = reinterpret_cast<uint32_t*>(P.hand);  // the 16 hand bytes, as in the row
        hand32[0] = m1;
        hand32[1] = m2;
        hand32[2] = m3;
        hand32[3] = m4;
        P.turn = (uint16_t)m5;  // turn u16, queen_placed u8, result u8
        P.qplaced = (uint8_t)(m5 >> 16);
        P.result = (uint8_t)(m5 >> 24);
        P.stun = (uint16_t)m6;
    }
}

// A loaded board's base fields -- everything load_position writes -- held in
// the group's registers: lane l keeps its 16-cell chunks l and (l < 2) 32 + l,
// the bitboard words l + 1 (l < 18) and metadata word l - 24 (24 <= l < 31;
// queen squares, turn, stun, hands, queen-placed, result).  restore_base puts
// them back after a move was applied on the board, so the successors of one
// parent read its row once.  Only load_position and apply_on_board write these
// fields; the later passes rebuild everything else of the board.
struct BaseRegs {
    u32x4 c0, c1;
    uint32_t occ, wt, bt, meta;
};
static_assert(offsetof(Pos, queen) % 4 == 0 && offsetof(Pos, turn) == offsetof(Pos, queen) + 4 &&
                  offsetof(Pos, stun) == offsetof(Pos, queen) + 6 && offsetof(Pos, hand) == offsetof(Pos, queen) + 8 &&
                  offsetof(Pos, qplaced) == offsetof(Pos, queen) + 24 &&
                  offsetof(Pos, result) == offsetof(Pos, queen) + 25 && offsetof(Pos, cell) % 16 == 0,
              "metadata words and cell chunks");

HW_INL void save_base(const Pos& P, BaseRegs& R, int lane) {  // after the barrier that follows the load
    const int l = gl(lane);
    const uint32_t* cell32 = reinterpret_cast<const uint32_t*>(P.cell);
    R.c0 = *reinterpret_cast<const u32x4*>(cell32 + 4 * l);
    u32x4 z = {0u, 0u, 0u, 0u};
    R.c1 = l < 34 - kW ? *reinterpret_cast<const u32x4*>(cell32 + 4 * (kW + l)) : z;
    R.occ = l < 18 ? P.occ[l + 1] : 0u;
    R.wt = l < 18 ? P.wt[l + 1] : 0u;
    R.bt = l < 18 ? P.bt[l + 1] : 0u;
    R.meta = (l >= 24 && l < 31) ? reinterpret_cast<const uint32_t*>(P.queen)[l - 24] : 0u;
}

HW_INL void restore_base(Pos& P, const BaseRegs& R, int lane) {
    const int l = gl(lane);
    uint32_t* cell32 = reinterpret_cast<uint32_t*>(P.cell);
    *reinterpret_cast<u32x4*>(cell32 + 4 * l) = R.c0;
    if (l < 34 - kW) *reinterpret_cast<u32x4*>(cell32 + 4 * (kW + l)) = R.c1;
    if (l < 18) {
        P.occ[l + 1] = R.occ;
        P.wt[l + 1] = R.wt;
        P.bt[l + 1] = R.bt;
    } else if (l >= 24 && l < 31) {
        reinterpret_cast<uint32_t*>(P.queen)[l - 24] = R.meta;
    }
}

// Ascending list of occupied cells (first 32) and per-word occupied-cell
// prefix counts.
HW_INL void build_occ_list(Pos& P, int lane) {
    const int l = gl(lane);
    uint32_t w = l < 18 ? P.occ[l + 1] : 0u;
    int base = grp_excl_scan(__popc(w));
    int total = grp_sum(__popc(w), lane);
    if (l < 18) P.occ_pre[l] = (uint16_t)base;
    int k = base;
    while (w && k < 32) {
        int b = __ffs(w) - 1;
        w &= w - 1;
        P.occ_cells[k] = (uint16_t)(l * 32 + b);
        k++;
    }
    if (l == 0) P.n_occ = total < 32 ? total : 32;
}

// index of occupied cell c in ascending cell order
HW_INL int occ_rank(const Pos& P, int c) {
    int w = c >> 5;
    return P.occ_pre[w] + __popc(P.occ[w + 1] & ((1u << (c & 31)) - 1u));
}

// occupied-neighbour direction mask of an occupied cell
HW_INL uint32_t nbo(const Pos& P, int c) {
    int r = occ_rank(P, c);
    return r < 32 ? (uint32_t)P.nbd[r] : nbr_bits(P.occ, c);
}

// On-grid neighbour directions of every board cell, one byte per cell (the
// grid6 bits), four cells per word; cells past the board have none.
struct GridBytes {
    uint32_t w[133];
};
constexpr GridBytes make_grid_bytes() {
    GridBytes g{};
    for (int c = 0; c < kCells; c++) {
        int r = c / kGrid, col = c % kGrid;
        uint32_t m = (col < 22 ? 1u : 0u) | (col < 22 && r > 0 ? 2u : 0u) | (r > 0 ? 4u : 0u) |
                     (col > 0 ? 8u : 0u) | (col > 0 && r < 22 ? 16u : 0u) | (r < 22 ? 32u : 0u);
        g.w[c >> 2] |= m << (8 * (c & 3));
    }
    return g;
}
static __constant__ GridBytes kGridBytes = make_grid_bytes();

// bits 0-3 of x to bits 0, 8, 16, 24 (x * 0x204081 puts bit k at 7k + 8k' for
// its four copies; bit k's copy at 8k is the only one on a byte's bit 0)
__device__ __forceinline__ uint32_t spread4(uint32_t x) { return (x * 0x00204081u) & 0x01010101u; }

// Ground-slide direction masks of the current occupancy (P.occ with zero
// pads) for the board rows of the hive grown by one row each way (every hex
// neighbour of an occupied cell lies in them; readers only look at occupied
// cells and their neighbours), the occupied-neighbour masks of the occupied
// cells (nbd, by rank) and the articulation test's adjacency rows (u1.adj).  A lane takes four cells c..c+3 (one word of
// sm): their neighbours in direction d are bits k + OFS(d) of the occupancy
// window starting at cell c - 23, spread to one byte per cell; the exit rule
// gm & ~n & (rotl6(n) ^ rotr6(n)) then runs on the four bytes at once.
HW_INL void build_cell_masks(Pos& P, int lane) {
    const int l = gl(lane);
    if (l < P.n_occ) {
        const int c = P.occ_cells[l];
        const uint64_t win = bit_window(P.occ, c - 23);  // bit k: cell c - 23 + k
        const uint32_t nm = ring_bits(win) & grid6(c);
        P.nbd[l] = (uint8_t)nm;
        // the articulation flood's dense adjacency row of vertex l (ranks
        // below kArtN): a neighbour's rank is l plus or minus the occupied
        // cells between it and c, counted in the same window
        const int N = min(P.n_occ, kArtN);
        if (l < N) {
            const uint32_t lo = (uint32_t)win, hi = (uint32_t)(win >> 24);
            const int up = __popc(lo & 0x7FFFFEu);    // cells c-22 .. c-1
            const int dn = __popc(hi & 0x1FFFFFu);    // cells c+1 .. c+21
            const int rk[6] = {l + 1, l - up, l - up - (int)(lo & 1u), l - 1, l + 1 + dn,
                               l + 1 + dn + (int)((hi >> 21) & 1u)};  // E NE NW W SW SE
            uint32_t a = 0;
#pragma unroll
            for (int d = 0; d < 6; d++)
                if (((nm >> d) & 1u) && rk[d] < N) a |= 1u << rk[d];
            P.u1.adj[l] = a;
        }
    }
    uint32_t rowbits = l < kGrid ? (word_field(P.occ, kGrid * l) & 0x7FFFFFu) : 0u;
    uint32_t rows = grp_ballot(rowbits != 0, lane);
    if (rows == 0) return;
    int r0 = __ffs(rows) - 1, r1 = 31 - __clz(rows);
    int rlo = r0 > 0 ? r0 - 1 : 0, rhi = r1 < kGrid - 1 ? r1 + 1 : kGrid - 1;
    const int g0 = (kGrid * rlo) >> 2, g1 = (kGrid * rhi + kGrid - 1) >> 2;
    uint32_t* sm4 = reinterpret_cast<uint32_t*>(P.sm);
    for (int g = g0 + l; g <= g1; g += kW) {
        const int lo = 4 * g - 23;
        const int wi = (lo >> 5) + 1, sh = lo & 31;
        uint64_t win = ((uint64_t)P.occ[wi] | ((uint64_t)P.occ[wi + 1] << 32)) >> sh;
        if (sh) win |= (uint64_t)P.occ[wi + 2] << (64 - sh);
        const uint32_t wl = (uint32_t)win, wh = (uint32_t)(win >> 32);
        uint32_t n = spread4((wl >> 24) & 15u) | (spread4((wl >> 1) & 15u) << 1) | (spread4(wl & 15u) << 2) |
                     (spread4((wl >> 22) & 15u) << 3) | (spread4((wh >> 13) & 15u) << 4) |
                     (spread4((wh >> 14) & 15u) << 5);
        const uint32_t gm = kGridBytes.w[g];
        n &= gm;
        const uint32_t rl = ((n << 1) & 0x3E3E3E3Eu) | ((n >> 5) & 0x01010101u);
        const uint32_t rr = ((n >> 1) & 0x1F1F1F1Fu) | ((n << 5) & 0x20202020u);
        sm4[g] = gm & ~n & (rl ^ rr);
    }
}
static_assert(sizeof(((Pos*)nullptr)->sm) >= 4 * 133, "sm holds whole words up to cell 531");

// Articulation points (articulation.cuh:34-168).  The reference runs one DFS
// from the lowest occupied cell, so its result is the articulation set of
// that cell's component (first 28 cells), empty when <= 2 cells are occupied.
// Here lane v floods the dense vertex graph with v removed; lane 31 floods
// with nothing removed to obtain the component C0 of vertex 0.  v is an
// articulation point iff v is in C0 and C0 \ {v} is not reached from a
// vertex of C0 \ {v}.
HW_INL void articulation(Pos& P, int lane) {
    const int l = gl(lane);
    int total = P.n_occ;
    int N = total < kArtN ? total : kArtN;
    if (l < 20) P.pin[l] = 0;
    __syncthreads();  // the adjacency rows written by build_cell_masks
    if (total <= 2) return;
    int v = l < N ? l : -1;
    uint32_t vbit = v >= 0 ? (1u << v) : 0u;
    uint32_t start;
    if (v == 0) {
        uint32_t a0 = P.u1.adj[0];
        start = a0 ? (a0 & (~a0 + 1u)) : 0u;
    } else {
        start = 1u;
    }
    uint32_t reach = 0;
    if (l < N || l == kW - 1) {
        // the flood's result is a set: frontier vertices are taken two at a
        // time (the second read repeats the first when only one is left)
        reach = start;
        uint32_t frontier = start;
        while (frontier) {
            const int i1 = __ffs(frontier) - 1;
            frontier &= frontier - 1;
            const int i2 = frontier ? __ffs(frontier) - 1 : i1;
            frontier &= frontier - 1;
            const uint32_t nb = (P.u1.adj[i1] | P.u1.adj[i2]) & ~reach & ~vbit;
            reach |= nb;
            frontier |= nb;
        }
    }
    uint32_t c0 = grp_shfl(reach, kW - 1, lane);
    bool is_ap = v >= 0 && ((c0 >> v) & 1u) && reach != (c0 & ~vbit);
    if (is_ap) {
        int c = P.occ_cells[v];
        if (P.hgt(c) == 1) atomicOr(&P.pin[(c >> 5) + 1], 1u << (c & 31));
    }
}

// ---------------------------------------------------------------- slides
// Ground-slide destinations of c (can_slide, move_gen.cuh:82-104): the
// destination is empty, exactly one of the two flanking cells is occupied;
// cell g counts as empty (the moving piece's origin).
__device__ __forceinline__ uint32_t slide_mask(const Pos& P, int c, int g) {
    uint32_t s = P.sm[c];
    uint32_t w = (uint32_t)(g - c + 23);
    if (w < 47u && ((kRingWin >> w) & 1ull)) {  // g may be a neighbour: recompute with g empty
        uint32_t gm = grid6(c);
        uint32_t n = nbr_bits(P.occ, c) & ~dir_bit_to(c, g, gm);
        s = gm & ~n & (rotl6(n) ^ rotr6(n));
    }
    return s;
}

// heights of the six neighbours (0 off-grid), 4 bits each: direction d at bits 4d..4d+3
__device__ __forceinline__ uint32_t nbr_heights(const Pos& P, int c, uint32_t gm) {
    uint32_t r = 0;
#pragma unroll
    for (int d = 0; d < 6; d++)
        if ((gm >> d) & 1u) r |= (uint32_t)(P.hgt(step(c, d)) & 15) << (4 * d);
    return r;
}
__device__ __forceinline__ int hof(uint32_t nh, int d) { return (int)((nh >> (4 * d)) & 15u); }
// both flanks of direction d strictly above height lvl (elevated gate, move_gen.cuh:659-667)
__device__ __forceinline__ bool gate_high(uint32_t nh, int d, int lvl) {
    return hof(nh, (d + 5) % 6) > lvl && hof(nh, (d + 1) % 6) > lvl;
}

// lane-private set helpers over an 18-word bitboard
__device__ __forceinline__ void set_clear(uint32_t* s) {  // 17 words: cells < 544
#pragma unroll
    for (int i = 0; i < 17; i++) s[i] = 0;
}
__device__ __forceinline__ bool set_insert(uint32_t* s, int c) {  // true if newly inserted
    uint32_t bit = 1u << (c & 31);
    return !(atomicOr(&s[c >> 5], bit) & bit);
}

// ---------------------------------------------------------------- generators
// Each writes destination cells into out[] in the reference's order and
// returns the count.

// gen_queen_moves :202-212 / gen_pillbug_moves :644-647
HW_INL int gen_step(const Pos& P, int c, uint16_t* out) {
    uint32_t m = slide_mask(P, c, c);
    int n = 0;
    while (m) {
        int d = __ffs(m) - 1;
        m &= m - 1;
        out[n++] = (uint16_t)step(c, d);
    }
    return n;
}

// Byte d of the 8-byte table {hi:lo} (one v_perm_b32; selector 0x0c = zero byte).
__device__ __forceinline__ uint32_t dir_byte(uint32_t hi, uint32_t lo, int d) {
    return __builtin_amdgcn_perm(hi, lo, 0x0c0c0c00u | (uint32_t)d);
}
// cell offset + 23 of direction d (24 1 0 22 45 46) and the opposite
// direction's bit 1 << ((d + 3) % 6) (8 16 32 1 2 4)
constexpr uint32_t kOfsLo = 24u | (1u << 8) | (0u << 16) | (22u << 24), kOfsHi = 45u | (46u << 8);
constexpr uint32_t kOppLo = 8u | (16u << 8) | (32u << 16) | (1u << 24), kOppHi = 2u | (4u << 8);

// gen_grasshopper_moves :228-245: over each occupied neighbour (directions
// in order), along the line to the first empty cell; no move when the line
// leaves the grid.  Row and column are stepped along (row / column deltas
// of direction d: nibble d of kDRow / kDCol, plus one).
constexpr uint32_t kDRow = 0x221001u, kDCol = 0x100122u;
// landing cell of a jump from c (row r0, column q0) over its occupied
// neighbour in direction d, or -1 when the line leaves the grid
HW_INL int hop_dest(const Pos& P, int c, int r0, int q0, int d) {
    const int dc = (int)dir_byte(kOfsHi, kOfsLo, d) - 23;
    const int dr = (int)((kDRow >> (4 * d)) & 15u) - 1, dq = (int)((kDCol >> (4 * d)) & 15u) - 1;
    int p = c + dc, r = r0 + dr, q = q0 + dq;  // occupied
    while (pb_get(P.occ, p)) {
        r += dr;
        q += dq;
        if ((unsigned)r >= (unsigned)kGrid || (unsigned)q >= (unsigned)kGrid) return -1;
        p += dc;
    }
    return p;
}
HW_INL int gen_hopper(const Pos& P, int c, uint16_t* out) {
    int n = 0;
    uint32_t m = nbo(P, c);
    const int r0 = row_of(c), q0 = c - r0 * kGrid;
    while (m) {
        const int d = __ffs(m) - 1;
        m &= m - 1;
        const int p = hop_dest(P, c, r0, q0, d);
        if (p >= 0) out[n++] = (uint16_t)p;
    }
    return n;
}

// FIFO breadth-first ant search (gen_ant_moves_with_perimeter :267-313,
// emit_ant_moves_with_perimeter :348-388): seeds in direction order, each
// dequeued cell expanded in direction order, ant lifted from c.
constexpr int kDirShift = 10;
constexpr int kCellMask = (1 << kDirShift) - 1;

// Slide exits of x, an empty neighbour of the lifted origin c in direction
// d of c, from its exits s with c occupied.  Only the exits b - 1, b, b + 1
// around b = d + 3 (the direction x -> c) change:
//   * exit b leads into c; its flanks are c's neighbours d + 1 and d + 5:
//     open iff exactly one of them is occupied (bit d of ox);
//   * exits b + 1 and b - 1 lead to c's neighbours d + 5 and d + 1; their
//     flank c turns empty, so an on-grid empty target is now open iff the
//     far flank is occupied, i.e. iff the exit was closed: ey / ez carry
//     "target on-grid and empty" at bit d.
__device__ __forceinline__ uint32_t lifted_exits(uint32_t s, int d, uint32_t ox, uint32_t ey, uint32_t ez) {
    const int b = d >= 3 ? d - 3 : d + 3;
    const int bh = b == 5 ? 0 : b + 1, bl = b == 0 ? 5 : b - 1;
    uint32_t r = s & ~((1u << b) | (1u << bh) | (1u << bl));
    r |= ((ox >> d) & 1u) << b;
    r |= ((ey >> d) & ~(s >> bh) & 1u) << bh;
    r |= ((ez >> d) & ~(s >> bl) & 1u) << bl;
    return r;
}

// A piece at c about to move: c's occupied / empty on-grid neighbour masks
// rotated so that bit d carries what lifted_exits needs for c's neighbour d.
struct Lift {
    int c;
    uint32_t ox, ey, ez;
};
HW_INL Lift lift_of(const Pos& P, int c) {
    const uint32_t oc = nbo(P, c), ec = grid6(c) & ~oc;
    return Lift{c, rotr6(oc) ^ rotl6(oc), rotl6(ec), rotr6(ec)};
}
// exits of the empty cell x = step(lf.c, d) with the piece at lf.c lifted
__device__ __forceinline__ uint32_t exits_next_to(const Pos& P, int x, int d, const Lift& lf) {
    return lifted_exits(P.sm[x], d, lf.ox, lf.ey, lf.ez);
}
// exits of an empty cell x with the piece at lf.c lifted (slide_mask(P, x,
// lf.c)): x is tested for adjacency to lf.c by its window position
// w = x - lf.c + 23 on the ring; its direction d from lf.c is read from w:
// the row r = (w + 1) / 23 and w + 1 - 20 r in {5 2 1 3 6 7} for d = 0..5.
__device__ __forceinline__ uint32_t exits_lifted(const Pos& P, int x, const Lift& lf) {
    uint32_t m = P.sm[x];
    const uint32_t w = (uint32_t)(x - lf.c + 23);
    if (w < 47u && ((kRingWin >> w) & 1ull)) {
        const uint32_t w1 = w + 1u, r = (w1 * 2850u) >> 16;
        const int d = (int)((0x54003120u >> (4u * (w1 - 20u * r))) & 15u);
        m = lifted_exits(m, d, lf.ox, lf.ey, lf.ez);
    }
    return m;
}

// exits_lifted for the ant search, as a lookup: the lifted exits of the
// origin's six neighbour cells are computed once per search and kept in 8
// bytes {hi:lo} by ring slot.  The window position w = x - c + 23 of c's
// neighbour in direction d is one of 24 1 0 22 45 46 (d = 0..5), and
// ((w * 19) >> 4) & 7 sends these to the distinct slots 4 1 0 2 5 6; x is a
// neighbour of c exactly when byte slot(w) of kRingW is w (slots 3 and 7 hold
// 0, whose own slot is 0, so no w matches them).
constexpr uint32_t kRingW[6] = {24, 1, 0, 22, 45, 46};
constexpr uint32_t ring_slot_of(uint32_t w) { return ((w * 19u) >> 4) & 7u; }
constexpr uint32_t kRingWLo = 0u | (1u << 8) | (22u << 16), kRingWHi = 24u | (45u << 8) | (46u << 16);
static_assert(ring_slot_of(24) == 4 && ring_slot_of(1) == 1 && ring_slot_of(0) == 0 && ring_slot_of(22) == 2 &&
                  ring_slot_of(45) == 5 && ring_slot_of(46) == 6,
              "ring slots: byte s of {kRingWHi:kRingWLo} is the window position of slot s");
__device__ __forceinline__ uint32_t ring_slot(uint32_t w) { return (__umul24(w, 19u) >> 4) & 7u; }
struct RingLift {
    int base;        // c - 23
    uint32_t lo, hi;  // lifted exits by ring slot
};
HW_INL RingLift ring_lift(const Pos& P, int c) {
    const Lift lf = lift_of(P, c);
    uint32_t t[2] = {0u, 0u};
#pragma unroll
    for (int d = 0; d < 6; d++) {
        const int x = c - 23 + (int)kRingW[d];
        const uint32_t e = (unsigned)x < (unsigned)kCells ? lifted_exits(P.sm[x], d, lf.ox, lf.ey, lf.ez) : 0u;
        const uint32_t s = ring_slot_of(kRingW[d]);
        t[s >> 2] |= e << (8 * (s & 3));
    }
    return RingLift{c - 23, t[0], t[1]};
}
// exits_lifted(P, x, lift_of(P, c)) for any cell x
__device__ __forceinline__ uint32_t exits_ring(const Pos& P, int x, const RingLift& rl) {
    const uint32_t w = (uint32_t)(x - rl.base), s = ring_slot(w);
    const uint32_t m = P.sm[x], lifted = __builtin_amdgcn_perm(rl.hi, rl.lo, 0x0c0c0c00u | s);
    return __builtin_amdgcn_perm(kRingWHi, kRingWLo, 0x0c0c0c00u | s) == w ? lifted : m;
}

// Queue entries are cell | (bit of the direction back to the parent) <<
// kDirShift: that exit leads to a visited cell and is skipped.  kStop: the
// search ends as soon as cell `stop` is discovered (*stopped set), leaving a
// prefix of the list that ends with it.  kLimit: the search also ends after
// `steps` expansions (the origin's own counts as one) with *next = the index
// of the next entry to expand and *rlo = the origin's lifted exits, so that
// ant_searches can take it from there; it is unfinished when *stopped is
// clear and *next < the returned length < cap.
template <bool kStop = false, bool kLimit = false>
HW_INL int gen_ant(const Pos& P, int c, uint16_t* out, int cap, uint32_t* seen, int stop = -1,
                   bool* stopped = nullptr, int steps = 0, int* next = nullptr, RingLift* rlo = nullptr) {
    set_clear(seen);
    set_insert(seen, c);
    const RingLift rl = ring_lift(P, c);
    if (kLimit) *rlo = rl;
    // queue by pointers: q = next free entry, h = next entry to expand
    uint16_t* q = out;
    const uint16_t* h = out;
    uint16_t* const end = out + cap;
    uint16_t* const roomy = out + (cap - 6);  // q <= roomy: every exit of a cell fits
    int cur = c;
    uint32_t back = 0;
    for (;;) {
        uint32_t m = exits_ring(P, cur, rl) & ~back;
        const int base = cur - 23;
        if (q <= roomy) {
            while (m) {
                const int d = __ffs(m) - 1;
                m &= m - 1;
                const int dest = base + (int)dir_byte(kOfsHi, kOfsLo, d);
                if (set_insert(seen, dest)) {
                    *q++ = (uint16_t)(dest | (dir_byte(kOppHi, kOppLo, d) << kDirShift));
                    if (kStop && dest == stop) {
                        *stopped = true;
                        return (int)(q - out);
                    }
                }
            }
        } else {
            while (m && q < end) {
                const int d = __ffs(m) - 1;
                m &= m - 1;
                const int dest = base + (int)dir_byte(kOfsHi, kOfsLo, d);
                if (set_insert(seen, dest)) {
                    *q++ = (uint16_t)(dest | (dir_byte(kOppHi, kOppLo, d) << kDirShift));
                    if (kStop && dest == stop) {
                        *stopped = true;
                        return (int)(q - out);
                    }
                }
            }
        }
        if (h >= q || q >= end) break;
        if (kLimit && --steps == 0) break;
        const uint32_t e = *h++;
        cur = (int)(e & kCellMask);
        back = e >> kDirShift;
    }
    if (kLimit) *next = (int)(h - out);
    return (int)(q - out);
}

// Long ant searches finished by the whole lane group of their position.  A
// search that gen_ant<kStop, true> left unfinished continues as gen_ant's
// FIFO taken up to five queued entries at a time, lane 6k + d expanding
// entry k of the batch in direction d (lanes 30, 31 idle).  A batch's
// entries are already in the queue, so expanding them together appends what
// expanding them one by one would, in the same order -- entry, then
// direction -- provided a cell reached from two entries of the batch is
// credited to the lower lane only: the lanes insert into the visited set
// together, and when a cell had two claimants the lower lane is made the
// winner whichever insert came first.  gen_ant's back-direction mask only
// skips visited cells, so it is not needed; the entries appended here carry
// no back bit.
//
// Lanes with `job` set hand in their search (origin c, list at
// P.u2.pool[off] with room cap and `len` entries of which the first `next`
// are expanded, visited set P.u1.sets[set], lifted exits rl) and get back the
// final length in m (and, with kStop, whether it stopped at `stop`).  Every
// lane of the group must call this.
constexpr bool kAntGroup = HW_ANT_GROUP != 0;
constexpr int kAntLaneSteps = HW_ANT_GROUP;  // expansions an ant lane makes before the group takes over
template <bool kStop = false>
HW_INL void ant_searches(Pos& P, int lane, bool job, int c, int off, int cap, int set, int len, int next,
                         RingLift rl, int stop, int& m, bool& stopped) {
    const int l = gl(lane);
    const int k = l / 6, d = l - 6 * k;
    const int ofs = (int)dir_byte(kOfsHi, kOfsLo, d) - 23;
    const uint32_t below = (1u << l) - 1u;
    uint32_t jobs = grp_ballot(job, lane);
    while (jobs) {
        const int j = __ffs(jobs) - 1;
        jobs &= jobs - 1;
        const int capj = grp_shfl(cap, j, lane);
        const RingLift rj{grp_shfl(c, j, lane) - 23, grp_shfl(rl.lo, j, lane), grp_shfl(rl.hi, j, lane)};
        uint16_t* out = P.u2.pool + grp_shfl(off, j, lane);
        uint32_t* seen = P.u1.sets[grp_shfl(set, j, lane)];
        int h = grp_shfl(next, j, lane), q = grp_shfl(len, j, lane);
        bool hit = false;
        while (h < q && q < capj && !hit) {
            const int np = min(5, q - h);
            bool cand = false;
            int dest = 0;
            if (k < np) {
                const int cur = (int)(out[h + k] & kCellMask);
                if ((exits_ring(P, cur, rj) >> d) & 1u) {  // open exits lead to on-grid cells
                    dest = cur + ofs;
                    cand = !((seen[dest >> 5] >> (dest & 31)) & 1u);
                }
            }
            hw_group_lockstep();  // every read of the set above precedes the inserts
            bool won = cand && set_insert(seen, dest);
            uint32_t lost = grp_ballot(cand && !won, lane);
            while (lost) {  // a cell with two claimants in the batch: the lower lane takes it
                const int dl = grp_shfl(dest, __ffs(lost) - 1, lane);
                const uint32_t same = grp_ballot(cand && dest == dl, lane);
                if (cand && dest == dl) won = l == __ffs(same) - 1;
                lost &= ~same;
            }
            const uint32_t wm = grp_ballot(won, lane);
            int nw = __popc(wm);
            const int rank = __popc(wm & below);
            if (kStop) {  // the list ends with `stop` once it is appended
                const uint32_t sb = grp_ballot(won && dest == stop, lane);
                if (sb) {
                    const int rs = __popc(wm & ((sb & (0u - sb)) - 1u));
                    if (q + rs < capj) {
                        nw = rs + 1;
                        hit = true;
                    }
                }
            }
            if (won && rank < nw && q + rank < capj) out[q + rank] = (uint16_t)dest;
            h += np;
            q = min(capj, q + nw);
            hw_group_lockstep();  // the next batch reads the entries written here
        }
        if (l == j) {
            m = q;
            stopped = hit;
        }
    }
}

// gen_spider_moves :397-431 (first occurrence over d1,d2,d3; at most 32)
HW_INL int gen_spider(const Pos& P, int c, uint16_t* out, uint32_t* got) {
    set_clear(got);
    int n = 0;
    const Lift lf = lift_of(P, c);
    uint32_t m1 = P.sm[c];
    // the step back (p2 == c, p3 == p1) is the exit opposite the arrival
    // direction: masked out instead of taken and skipped
    while (m1) {
        int d1 = __ffs(m1) - 1;
        m1 &= m1 - 1;
        int p1 = c - 23 + (int)dir_byte(kOfsHi, kOfsLo, d1);
        uint32_t m2 = exits_next_to(P, p1, d1, lf) & ~dir_byte(kOppHi, kOppLo, d1);
        while (m2) {
            int d2 = __ffs(m2) - 1;
            m2 &= m2 - 1;
            int p2 = p1 - 23 + (int)dir_byte(kOfsHi, kOfsLo, d2);
            uint32_t m3 = exits_lifted(P, p2, lf) & ~dir_byte(kOppHi, kOppLo, d2);
            while (m3) {
                int d3 = __ffs(m3) - 1;
                m3 &= m3 - 1;
                int p3 = p2 - 23 + (int)dir_byte(kOfsHi, kOfsLo, d3);
                if (p3 == c) continue;
                if (n < 32 && set_insert(got, p3)) out[n++] = (uint16_t)p3;
            }
        }
    }
    return n;
}

// gen_beetle_moves :468-502
HW_INL int gen_beetle(const Pos& P, int c, uint16_t* out) {
    uint32_t gm = grid6(c);
    uint32_t nh = nbr_heights(P, c, gm);
    uint32_t sm = slide_mask(P, c, c);
    int below = P.hgt(c) - 1;
    int n = 0;
    for (int d = 0; d < 6; d++) {
        if (!((gm >> d) & 1u)) continue;
        int mh = max(hof(nh, d), below);
        bool ok;
        if (mh > 0) ok = !gate_high(nh, d, mh);
        else ok = (sm >> d) & 1u;
        if (ok) out[n++] = (uint16_t)step(c, d);
    }
    return n;
}

// gen_ladybug_moves :538-596 (first occurrence over d1,d2,d3; at most 32)
HW_INL int gen_ladybug(const Pos& P, int c, uint16_t* out, uint32_t* got) {
    set_clear(got);
    int n = 0;
    uint32_t g0 = grid6(c);
    uint32_t nh0 = nbr_heights(P, c, g0);
    uint32_t o0 = nbo(P, c);
    int hc = P.hgt(c);
    for (int d1 = 0; d1 < 6; d1++) {
        if (!((o0 >> d1) & 1u)) continue;
        int p1 = step(c, d1);
        if (gate_high(nh0, d1, max(hc - 1, hof(nh0, d1)))) continue;
        uint32_t nh1 = nbr_heights(P, p1, grid6(p1));
        uint32_t o1 = nbo(P, p1);
        int hp1 = P.hgt(p1);
        for (int d2 = 0; d2 < 6; d2++) {
            if (!((o1 >> d2) & 1u)) continue;
            int p2 = step(p1, d2);
            if (p2 == c) continue;
            if (gate_high(nh1, d2, max(hp1, hof(nh1, d2)))) continue;
            uint32_t g2 = grid6(p2);
            uint32_t nh2 = nbr_heights(P, p2, g2);
            uint32_t o2 = nbo(P, p2);
            int mh3 = P.hgt(p2);
            for (int d3 = 0; d3 < 6; d3++) {
                if (!((g2 >> d3) & 1u) || ((o2 >> d3) & 1u)) continue;
                int p3 = step(p2, d3);
                if (p3 == c || p3 == p1) continue;
                if (gate_high(nh2, d3, mh3)) continue;
                if (n < 32 && set_insert(got, p3)) out[n++] = (uint16_t)p3;
            }
        }
    }
    return n;
}

// gen_mosquito_moves :907-1008: beetle when stacked; otherwise the union, in
// order Q/P, A, G, S, B, L, of the abilities of adjacent non-mosquito top
// pieces, first occurrence kept (the reference caps it at 128; it has at
// most 64 entries).  Each sub-list is generated into the free tail of out[]
// and merged in place (merge write index never passes the read index);
// kMosqRoom slots hold the union so far (<= 64) and a sub-list (<= 32), and
// a union past 64 entries (no state built by init/apply has one) stops the
// merging before a sub-list could run past the room.
template <bool kStop = false>
HW_INL int gen_mosquito(const Pos& P, int c, uint16_t* out, uint32_t* tmpset, uint32_t* unionset, int stop = -1,
                        bool* stopped = nullptr) {
    if (P.hgt(c) > 1) return gen_beetle(P, c, out);
    uint32_t gm = grid6(c);
    uint32_t om = nbo(P, c);
    uint32_t has = 0;
    for (int d = 0; d < 6; d++)
        if ((om >> d) & 1u) {
            int t = P.tp(step(c, d)) & 15;
            if (t != PT_M) has |= 1u << t;
        }
    (void)gm;
    set_clear(unionset);
    int n = 0;
    for (int k = 0; k < 6 && n <= kMosqRoom - 32; k++) {
        uint16_t* tail = out + n;
        int m = 0;
        switch (k) {
            case 0: if (has & ((1u << PT_Q) | (1u << PT_P))) m = gen_step(P, c, tail); break;
            case 1: if (has & (1u << PT_A)) m = gen_ant<kStop>(P, c, tail, kMosqRoom - n, tmpset, stop, stopped); break;
            case 2: if (has & (1u << PT_G)) m = gen_hopper(P, c, tail); break;
            case 3: if (has & (1u << PT_S)) m = gen_spider(P, c, tail, tmpset); break;
            case 4: if (has & (1u << PT_B)) m = gen_beetle(P, c, tail); break;
            case 5: if (has & (1u << PT_L)) m = gen_ladybug(P, c, tail, tmpset); break;
        }
        int w = n;
        for (int i = 0; i < m; i++) {
            int x = tail[i] & kCellMask;
            if (set_insert(unionset, x) && w < kMosqRoom) out[w++] = (uint16_t)x;
        }
        n = w;
    }
    return n;
}

// Throws by the pillbug-ability actor at a (gen_pillbug_throws :691-740):
// targets in direction order, each to the empty drop cells in direction order.
HW_INL int gen_throws(const Pos& P, int a, uint16_t* from, uint16_t* to, uint8_t* pt) {
    int n = 0;
    uint32_t ga = grid6(a);
    uint32_t nha = nbr_heights(P, a, ga);
    int ph = P.hgt(a);
    uint32_t oa = nbo(P, a);
    for (int dt = 0; dt < 6; dt++) {
        if (!((oa >> dt) & 1u)) continue;
        int t = step(a, dt);
        if (P.hgt(t) != 1) continue;
        if (P.stun != 0xFFFF && (int)P.stun == t) continue;
        if (pb_get(P.pin, t)) continue;
        int back = (dt + 3) % 6;  // direction from the target to the actor
        uint32_t gt = grid6(t);
        int lift = max(P.hgt(t) - 1, ph);
        int cwh = ((gt >> ((back + 5) % 6)) & 1u) ? P.hgt(step(t, (back + 5) % 6)) : 0;
        int ccwh = ((gt >> ((back + 1) % 6)) & 1u) ? P.hgt(step(t, (back + 1) % 6)) : 0;
        if (cwh > lift && ccwh > lift) continue;
        int tp = P.tp(t) & 15;
        for (int dd = 0; dd < 6; dd++) {
            if (!((ga >> dd) & 1u) || dd == dt || ((oa >> dd) & 1u)) continue;
            if (gate_high(nha, dd, ph) || n >= kThrowCap) continue;
            from[n] = (uint16_t)t;
            to[n] = (uint16_t)step(a, dd);
            pt[n] = (uint8_t)tp;
            n++;
        }
    }
    return n;
}

__device__ __forceinline__ bool touches_top_pillbug(const Pos& P, int c) {
    uint32_t m = nbo(P, c);
    while (m) {
        int d = __ffs(m) - 1;
        m &= m - 1;
        if ((P.tp(step(c, d)) & 15) == PT_P) return true;
    }
    return false;
}

__device__ __forceinline__ int type_capacity(int t) {
    return t == PT_A ? kAntCap : t == PT_M ? kMosqRoom : (t == PT_S || t == PT_L) ? 32 : 6;
}
__device__ __forceinline__ int type_sets(int t) {
    return t == PT_M ? 2 : (t == PT_A || t == PT_S || t == PT_L) ? 1 : 0;
}

// ---------------------------------------------------------------- placement
// Placement cells (find_placement_positions :1064-1140) are computed as a
// bit-parallel neighbourhood expression over board words (lane w < 18 owns
// word w) from nbr_union_word below.

// kGridMask.m[d][w]: cells of board word w whose d-neighbour is on the grid
struct GridMasks {
    uint32_t m[6][18];
};
constexpr GridMasks make_grid_masks() {
    GridMasks g{};
    for (int c = 0; c < kCells; c++) {
        int r = c / kGrid, col = c % kGrid;
        bool ok[6] = {col < 22, col < 22 && r > 0, r > 0, col > 0, col > 0 && r < 22, r < 22};
        for (int d = 0; d < 6; d++)
            if (ok[d]) g.m[d][c >> 5] |= 1u << (c & 31);
    }
    return g;
}
static __constant__ GridMasks kGridMask = make_grid_masks();

// kEdgeMask.m[w]: cells of board word w on the grid's border (row or column 0 or 22)
struct EdgeMask {
    uint32_t m[18];
};
constexpr EdgeMask make_edge_mask() {
    EdgeMask e{};
    for (int c = 0; c < kCells; c++) {
        const int r = c / kGrid, col = c % kGrid;
        if (r == 0 || r == kGrid - 1 || col == 0 || col == kGrid - 1) e.m[c >> 5] |= 1u << (c & 31);
    }
    return e;
}
static __constant__ EdgeMask kEdgeMask = make_edge_mask();

// cells of board word w with an on-grid neighbour that is set in pb
HW_INL uint32_t nbr_union_word(const uint32_t* pb, int w) {
    uint32_t r = 0;
#pragma unroll
    for (int d = 0; d < 6; d++) r |= word_field(pb, 32 * w + win_ofs(d) - 23) & kGridMask.m[d][w];
    return r;
}

}  // namespace hw
