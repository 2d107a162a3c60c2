// hive_engine.hip -- HIP kernels and the C-ABI of the batched Hive engine.
//
// Launch model: the per-position kernels run one 64-lane wavefront per
// position (workgroup = one wave, LDS board from hive_wave.hpp); the
// byte-level state kernels (init / apply / result) run one lane per state or
// per 16-byte chunk.  Every entry point takes device pointers, sizes and the
// caller's hipStream_t and returns a hipError_t code; nothing allocates.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hive_gpu.h"
#include "hive_leaf.hpp"
#include "hive_phases.hpp"

using namespace hw;

namespace {

// ---------------------------------------------------------------- state bytes
// init_state (hive_state.cuh:454-492) over a zero row: every byte of the
// row is written, one 16-byte chunk per lane.
__global__ void k_init_states(uint4* __restrict__ states, int64_t chunks, int mask) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= chunks) return;
    int k = (int)(i % (kStateBytes / 16));
    uint4 v = make_uint4(0, 0, 0, 0);
    if (k == OFF_QUEEN / 16) {  // bytes 3392..3407: queen cells, hands
        uint32_t x = (mask & 1) ? 1u : 0u, l = (mask & 2) ? 1u : 0u, p = (mask & 4) ? 1u : 0u;
        uint32_t hand_lo = 1u | (3u << 8) | (3u << 16) | (2u << 24);  // Q A G S
        uint32_t hand_hi = 2u | (x << 8) | (l << 16) | (p << 24);      // B M L P
        v = make_uint4(0xFFFFFFFFu, hand_lo, hand_hi, hand_lo);
    } else if (k == OFF_QUEEN / 16 + 1) {  // bytes 3408..3423
        uint32_t x = (mask & 1) ? 1u : 0u, l = (mask & 2) ? 1u : 0u, p = (mask & 4) ? 1u : 0u;
        uint32_t hand_hi = 2u | (x << 8) | (l << 16) | (p << 24);
        v = make_uint4(hand_hi, 0u /*turn, qplaced, result*/, 0xFFFFu /*stun; centre 0*/, 0u);
    }
    states[i] = v;
}

__global__ void k_apply_moves(uint8_t* __restrict__ states, const uint8_t* __restrict__ moves, int64_t B) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B) return;
    const uint8_t* m = moves + 6 * i;
    RowView v{states + i * kStateBytes};
    v.apply(m[0], m[1], m[2] | (m[3] << 8), m[4] | (m[5] << 8));
}

__global__ void k_check_results(const uint8_t* __restrict__ states, int64_t B, int32_t* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B) out[i] = states[i * kStateBytes + OFF_RESULT];
}

// ---------------------------------------------------------------- positions
// Two positions per 64-lane workgroup (lane groups of kW = 32).  A group
// whose item index is past the end works on the last item and writes
// nothing, so that both groups reach every barrier.
__device__ __forceinline__ int64_t item_of(int64_t n, bool& live) {
    const int64_t i = (int64_t)blockIdx.x * kPosPerWave + (threadIdx.x >> 5);
    live = i < n;
    return live ? i : n - 1;
}

// Processing order by turn.  A position's work grows with the pieces on the
// board, which follow the turn; a wave pays for the longer of its two
// positions' searches, and the launch ends with its longest waves.  So a
// launch can take its positions in buckets of 4 turns, latest turns first:
// k_order_buckets appends each position's index to the list of its bucket
// (lists[b * B ...], counts[b]), and k_legal<.., true> maps its item s to
// the s-th index of the concatenated lists.  Outputs are written at each
// position's own row, so the order changes no result.  The workspace holds
// two count arrays used in turn: a call counts into the one that is zero
// and clears the other (the previous call's, whose readers have finished
// on the same stream), so no launch is spent clearing.
// A workgroup takes kOrderPer positions (kOrderPer / 256 per thread, their
// turns loaded together), so the bucket offsets cost one global atomic per
// bucket per kOrderPer positions.
constexpr int kOrderBuckets = 32, kOrderShift = 2;  // buckets of 4 turns, turn >= 124 in the last
constexpr int kOrderPer = 1024, kOrderEach = kOrderPer / 256;
__global__ __launch_bounds__(256) void k_order_buckets(const uint8_t* __restrict__ states, int64_t B,
                                                       int32_t* __restrict__ counts, int32_t* __restrict__ clear,
                                                       int32_t* __restrict__ lists) {
    __shared__ int cnt[kOrderBuckets], base[kOrderBuckets];
    if (threadIdx.x < kOrderBuckets) cnt[threadIdx.x] = 0;
    if (blockIdx.x == 0 && threadIdx.x < kOrderBuckets) clear[threadIdx.x] = 0;
    int turn[kOrderEach];
#pragma unroll
    for (int k = 0; k < kOrderEach; k++) {
        const int64_t i = (int64_t)blockIdx.x * kOrderPer + k * 256 + threadIdx.x;
        turn[k] = i < B ? *reinterpret_cast<const uint16_t*>(states + i * kStateBytes + OFF_TURN) : -1;
    }
    __syncthreads();
    int b[kOrderEach], r[kOrderEach];
#pragma unroll
    for (int k = 0; k < kOrderEach; k++) {
        b[k] = turn[k] < 0 ? -1 : min(turn[k] >> kOrderShift, kOrderBuckets - 1);
        r[k] = b[k] >= 0 ? atomicAdd(&cnt[b[k]], 1) : 0;
    }
    __syncthreads();
    if (threadIdx.x < kOrderBuckets)
        base[threadIdx.x] = cnt[threadIdx.x] ? atomicAdd(&counts[threadIdx.x], cnt[threadIdx.x]) : 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kOrderEach; k++) {
        const int64_t i = (int64_t)blockIdx.x * kOrderPer + k * 256 + threadIdx.x;
        if (b[k] >= 0 && base[b[k]] + r[k] < B) lists[(int64_t)b[k] * B + base[b[k]] + r[k]] = (int32_t)i;
    }
}

// item s of the ordered launch (buckets from the latest turns down): lane
// k < 32 of the group holds the count of bucket 31 - k and its exclusive
// prefix; the item's bucket is the last one whose prefix is <= s.  32-bit
// index math (the entry point takes B < 2^31); the result is kept inside
// the batch even for a workspace used against its contract.
__device__ __forceinline__ uint32_t ordered_item(int s, const int32_t* __restrict__ counts,
                                                 const int32_t* __restrict__ lists, int B, int lane) {
    static_assert(kOrderBuckets == kW, "one bucket per lane of the group");
    const int k = gl(lane);
    const int c = counts[kOrderBuckets - 1 - k];
    const int excl = grp_excl_scan(c);
    const uint32_t le = grp_ballot(excl <= s, lane);  // lane 0's prefix is 0 <= s
    const int j = 31 - __clz(le);  // prefixes are non-decreasing: the highest lane with excl <= s
    const int start = grp_shfl(excl, j, lane);
    const uint32_t last = (uint32_t)(B - 1);
    const uint32_t off = min((uint32_t)max(s - start, 0), last);
    const uint32_t p = (uint32_t)lists[(size_t)(uint32_t)(kOrderBuckets - 1 - j) * (uint32_t)B + off];
    return min(p, last);
}

// 6 waves per SIMD: the register cap (80 VGPRs, a few bytes of spill) pays
// for itself, the kernel is bound by issue and latency, not by registers
template <bool WithMoves, bool WithFeat, bool WithAct, bool Ordered = false>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(6))) void k_legal(const uint8_t* __restrict__ states, int64_t B,
                                              uint8_t* __restrict__ moves_out, int32_t* __restrict__ n_out,
                                              float* __restrict__ feat_out, int32_t* __restrict__ act_out,
                                              const int32_t* __restrict__ counts = nullptr,
                                              const int32_t* __restrict__ lists = nullptr) {
    __shared__ Pos PS[kPosPerWave];
    bool live;
    int64_t pos = item_of(B, live);
    if (Ordered) pos = ordered_item((int)pos, counts, lists, (int)B, threadIdx.x);
    run_legal<WithMoves, WithFeat, WithAct>(PS[threadIdx.x >> 5], states + pos * kStateBytes, threadIdx.x,
                                            live ? moves_out + pos * (kMaxLegal * 6) : nullptr,
                                            live ? n_out + pos : nullptr,
                                            WithFeat && live ? feat_out + pos * kFeat : nullptr,
                                            WithAct && live ? act_out + pos * kMaxLegal : nullptr);
}

__global__ __launch_bounds__(64) void k_extract_features(const uint8_t* __restrict__ states,
                                                         const uint8_t* __restrict__ moves,
                                                         const int32_t* __restrict__ num_legal, int64_t B,
                                                         float* __restrict__ feat_out) {
    __shared__ Pos PS[kPosPerWave];
    __shared__ ListSets XS[kPosPerWave];
    bool live;
    const int64_t pos = item_of(B, live);
    run_extract(PS[threadIdx.x >> 5], XS[threadIdx.x >> 5], states + pos * kStateBytes,
                moves + pos * (kMaxLegal * 6), num_legal[pos], threadIdx.x, live ? feat_out + pos * kFeat : nullptr);
}

// legal_moves_to_actions_kernel (game_logic.cu:811-835) / compute_centroids_kernel
// (state_encoder.cuh:982-996): centroid over the occupied cells, one lane per list slot.
__global__ __launch_bounds__(64) void k_actions(const uint8_t* __restrict__ states,
                                                const uint8_t* __restrict__ moves,
                                                const int32_t* __restrict__ num_legal, int64_t B,
                                                int32_t* __restrict__ act_out, int32_t* __restrict__ centroid_out) {
    __shared__ Pos PS[kPosPerWave];
    const int lane = threadIdx.x;
    const int l = gl(lane);
    bool live;
    const int64_t pos = item_of(B, live);
    Pos& P = PS[lane >> 5];
    const uint8_t* S = states + pos * kStateBytes;
    const uint32_t* W = reinterpret_cast<const uint32_t*>(S + OFF_OCC);
    if (l < 18) P.occ[l + 1] = W[l];
    int n = 0;
    if (act_out) {
        n = num_legal[pos];
        n = n < 0 ? 0 : (n > kMaxLegal ? kMaxLegal : n);
    }
    __syncthreads();
    build_occ_list(P, lane);
    __syncthreads();
    int cq, cr;
    centroid(P, lane, cq, cr);
    if (centroid_out && live && l == 0) {
        centroid_out[2 * pos] = cq;
        centroid_out[2 * pos + 1] = cr;
    }
    if (act_out && live) list_actions(moves + pos * (kMaxLegal * 6), n, cq, cr, act_out + pos * kMaxLegal, lane);
}

// a zero state and move for rows that reference no valid (root, move)
__device__ __attribute__((aligned(16))) const uint8_t kZeroRow[kStateBytes] = {};

// rows of successor features per lane group: consecutive rows of one root
// share the root's load
constexpr int kSuccRows = 8;
constexpr int64_t kSuccGrid = 16384;  // workgroups of the successor kernels (they stride beyond)
// register budget of the successor kernels, by index type: the 32-bit row
// arithmetic fits 6 waves per SIMD (80 VGPRs, no spills; the LDS boards of
// 24 workgroups fill a CU's 160 KB), the 64-bit one 5 (96 VGPRs; at 80 it
// spills); left alone the row loop takes ~109
template <typename Ix>
constexpr int kSuccWaves = sizeof(Ix) == 4 ? 6 : 5;

// Row blocks of R rows: lane group q of the grid takes blocks q,
// q + 2 * gridDim.x, ... one row after another, as one stream (a root's
// board carries over a block boundary).  R = kSuccRows when every lane group
// of the grid has that many rows to do, fewer when the rows are few (down to
// one row per group: the count is known only on the device, and a short
// batch is bound by the latency of each group's rows in series, not by the
// board loads that longer runs share).  The loop count is uniform over the
// workgroup: both groups run while the first group's block is in range.
template <typename Ix>
HW_INL void successor_stream(const uint8_t* __restrict__ states, const uint8_t* __restrict__ legal,
                             const int64_t* __restrict__ a2r, const int64_t* __restrict__ midx, Ix N,
                             int64_t num_roots, float* __restrict__ feat_out) {
    __shared__ Pos PS[kPosPerWave];
    const int grp = threadIdx.x >> 5;
    const Ix groups = (Ix)kPosPerWave * (Ix)gridDim.x;
    const Ix per = (N + groups - 1) / groups;
    const int R = per < 1 ? 1 : (per > kSuccRows ? kSuccRows : (int)per);
    const Ix blocks = (N + R - 1) / R;
    SuccessorStream st;
    for (Ix p = blockIdx.x; kPosPerWave * p < blocks; p += gridDim.x) {
        for (int k = 0; k < R; k++) {
            const int lane = hw_opaque(threadIdx.x);
            const Ix i = (kPosPerWave * p + grp) * R + k;
            successor_row<Ix>(PS[grp], st, states, legal, a2r, midx, i, N, num_roots, kZeroRow, lane, feat_out);
        }
    }
}

// 32-bit row arithmetic is exact when every state, move and feature offset of
// the batch (rows < rows_cap, roots < num_roots) stays below 2^32
inline bool successor_narrow(int64_t rows_cap, int64_t num_roots) {
    return rows_cap >= 0 && num_roots >= 0 && rows_cap <= ((int64_t)1 << 32) / kFeat &&
           num_roots <= ((int64_t)1 << 32) / kStateBytes && num_roots <= ((int64_t)1 << 32) / (kMaxLegal * 6);
}

// fnn_successor_features_kernel (game_logic.cu:182-229): kSuccRows (root, move)
// rows per lane group, two groups per wave, the grid striding over the rows.
template <typename Ix>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(kSuccWaves<Ix>))) void k_successor_features(const uint8_t* __restrict__ states,
                                                           const uint8_t* __restrict__ legal,
                                                           const int64_t* __restrict__ a2r,
                                                           const int64_t* __restrict__ midx, int64_t N,
                                                           int64_t num_roots, float* __restrict__ feat_out) {
    successor_stream<Ix>(states, legal, a2r, midx, (Ix)N, num_roots, feat_out);
}

__global__ __launch_bounds__(64) void k_queen_escape(const uint8_t* __restrict__ states, int64_t B,
                                                     uint8_t* __restrict__ out) {
    __shared__ Pos PS[kPosPerWave];
    bool live;
    const int64_t pos = item_of(B, live);
    bool esc = run_queen_escape(PS[threadIdx.x >> 5], states + pos * kStateBytes, threadIdx.x);
    if (live && gl(threadIdx.x) == 0) out[pos] = esc ? 1 : 0;
}

// Surround count of the queen cell q (0xFFFF: unplaced, count 0; other
// cells clamped to the board) on the board after a move: occupied on-grid
// neighbours, the heights read from the LDS board with the move's effect
// added (dfrom loses a piece, dto gains one; -1: none).
HW_INL int surround_after(const Pos& P, int q, int dfrom, int dto) {
    if (q == 0xFFFF) return 0;
    q = q < 0 ? 0 : (q >= kCells ? kCells - 1 : q);
    const uint32_t gm = grid6(q);
    int k = 0;
    for (int d = 0; d < 6; d++) {
        if (!((gm >> d) & 1u)) continue;
        const int nb = step(q, d);
        k += P.hgt(nb) - (nb == dfrom ? 1 : 0) + (nb == dto ? 1 : 0) > 0 ? 1 : 0;
    }
    return k;
}

// The reserve-slot qualification of the Gumbel root candidates
// (fnn_mcts_orchestrator.py:338-378): legal child k of root r qualifies when
// its move raises the surround count of the opponent's queen (the child's
// side to move) and, with immobile_only, that side then has no queen escape
// (has_queen_escape_move, move_gen.cuh:771-821).  One lane group per root:
// its lanes take the slots and work each move's effect on the heights and on
// the queen's cell out from the root's board, as apply_move makes it; then
// the qualifying children are built on the board one after another (the
// root's board restored from registers) for the escape test.  Both groups of
// a workgroup run as many children as the busier one (barriers); a group's
// extra turns run a PASS and change nothing.  qual[r][k] = 1 or 0, all 256
// slots written.
//
// With cand: the root's candidate row as well (fnn_mcts_orchestrator.py:
// 411-444): `reserve` columns of qualifying slots by prior (-1 past the
// qualifying count), then the other columns of the row from every slot that
// is legal (and allowed) and not reserved, by prior, the rest (reserved and
// illegal slots, ranked at -1e30) after them; every ranking stable (ties to
// the lower slot), one group-wide argmax per column.
__device__ __forceinline__ void group_argmax(float v, int idx, int lane, float& bv, int& bi) {
#pragma unroll
    for (int o = 1; o < kW; o <<= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int oi = __shfl_xor(idx, o, 64);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    bv = v;
    bi = idx;
}
HW_INL void candidate_row(const uint32_t* keep, const uint32_t* valid, const float* __restrict__ pr, int k,
                          int reserve, int lane, int32_t* __restrict__ out) {
    const int l = gl(lane);
    const uint32_t bit = 1u << l;
    float p[kMaxLegal / kW];
    uint32_t chosen[kMaxLegal / kW];
    int nq = 0;
#pragma unroll
    for (int c = 0; c < kMaxLegal / kW; c++) {
        p[c] = pr[l + kW * c];
        chosen[c] = 0u;
        nq += __popc(keep[c]);
    }
    const int rpg = nq < reserve ? nq : reserve;  // reserve columns that hold a slot
    for (int pass = 0; pass < 2; pass++) {
        const int cols = pass == 0 ? reserve : k - reserve;
        uint32_t taken[kMaxLegal / kW];
#pragma unroll
        for (int c = 0; c < kMaxLegal / kW; c++) taken[c] = 0u;
        for (int j = 0; j < cols; j++) {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int c = 0; c < kMaxLegal / kW; c++) {
                if (taken[c] & bit) continue;
                const bool in = (pass == 0 ? keep[c] : (valid[c] & ~chosen[c])) & bit;
                const float v = in ? p[c] : -1e30f;
                const int idx = l + kW * c;
                if (v > bv || (v == bv && idx < bi)) {
                    bv = v;
                    bi = idx;
                }
            }
            group_argmax(bv, bi, lane, bv, bi);
#pragma unroll
            for (int c = 0; c < kMaxLegal / kW; c++)
                if (c == bi / kW) {
                    taken[c] |= 1u << (bi % kW);
                    if (pass == 0 && j < rpg) chosen[c] |= 1u << (bi % kW);
                }
            if (l == 0 && out) out[pass == 0 ? j : reserve + j] = (pass == 0 && j >= rpg) ? -1 : bi;
        }
    }
}

__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(5))) void k_reserve_qualify(
    const uint8_t* __restrict__ states, const uint8_t* __restrict__ legal, const int32_t* __restrict__ nlegal,
    int64_t B, int immobile, uint8_t* __restrict__ qual, const uint8_t* __restrict__ allowed,
    const float* __restrict__ priors, int k, int reserve, int32_t* __restrict__ cand) {
    __shared__ Pos PS[kPosPerWave];
    bool live;
    const int64_t r = item_of(B, live);
    Pos& P = PS[threadIdx.x >> 5];
    const int lane = threadIdx.x, l = gl(lane);
    const uint8_t* S = states + r * kStateBytes;
    load_position(P, S, lane);
    int n = nlegal[r];
    n = n < 0 ? 0 : (n > kMaxLegal ? kMaxLegal : n);
    __syncthreads();
    BaseRegs R;
    save_base(P, R, lane);
    const int opp = (P.turn & 1) ^ 1;
    const int q0 = P.queen[opp];
    const int before = surround_after(P, q0, -1, -1);
    const uint8_t* M = legal + r * (kMaxLegal * 6);
    // keep: the qualifying slots (by the count); pending: those still to be
    // tested for an escape; both one 32-slot word per chunk, group-uniform
    uint32_t keep[kMaxLegal / kW], pending[kMaxLegal / kW];
    int count = 0;
#pragma unroll
    for (int c = 0; c < kMaxLegal / kW; c++) {
        const int k = l + kW * c;
        bool q = false;
        if (k < n) {
            const uint8_t* m = M + 6 * k;
            const int type = m[0], pt = m[1], from = m[2] | (m[3] << 8), to = m[4] | (m[5] << 8);
            int dfrom = -1, dto = -1, qc = q0;
            if (type == MV_PLACE) {
                if (to < kCells && pt >= PT_Q && pt <= PT_P && P.hgt(to) < 5) dto = to;
            } else if (type == MV_MOVE) {
                if (from < kCells && to < kCells && P.hgt(from) > 0 && P.hgt(from) <= 5 && P.hgt(to) < 5) {
                    dfrom = from;
                    dto = to;
                    const int b = P.tp(from);
                    if ((b & 15) == PT_Q && ((b >> 4) & 1) == opp) qc = to;  // a thrown queen
                }
            }
            q = surround_after(P, qc, dfrom, dto) > before;
        }
        keep[c] = grp_ballot(q, lane);
        pending[c] = immobile ? keep[c] : 0u;
        count += immobile ? __popc(keep[c]) : 0;
    }
    // the workgroup's number of turns: the busier group's
    const int other = __shfl(count, (lane + kW) & 63, 64);
    const int turns = count > other ? count : other;
    for (int j = 0; j < turns; j++) {
        int slot = -1;
#pragma unroll
        for (int c = 0; c < kMaxLegal / kW; c++)
            if (slot < 0 && pending[c]) slot = kW * c + __ffs(pending[c]) - 1;
        restore_base(P, R, lane);
        __syncthreads();
        if (l == 0) {  // the escape test reads no result: the apply skips the ring test
            if (slot >= 0) {
                const uint8_t* m = M + 6 * slot;
                apply_on_board<false>(P, S, m[0], m[1], m[2] | (m[3] << 8), m[4] | (m[5] << 8));
            } else {
                apply_on_board<false>(P, S, MV_PASS, 0, 0, 0);  // a turn with nothing left to test
            }
        }
        __syncthreads();
        build_occ_list(P, lane);
        __syncthreads();
        build_cell_masks(P, lane);
        articulation(P, lane);
        __syncthreads();
        const bool esc = queen_escape(P, lane);
        if (slot >= 0) {
#pragma unroll
            for (int c = 0; c < kMaxLegal / kW; c++)
                if (c == slot / kW) {
                    pending[c] &= ~(1u << (slot % kW));
                    if (esc) keep[c] &= ~(1u << (slot % kW));
                }
        }
        __syncthreads();
    }
    if (live && qual) {
        uint8_t* out = qual + r * kMaxLegal;
#pragma unroll
        for (int c = 0; c < kMaxLegal / kW; c++) out[l + kW * c] = (uint8_t)((keep[c] >> l) & 1u);
    }
    if (cand) {
        uint32_t valid[kMaxLegal / kW];
#pragma unroll
        for (int c = 0; c < kMaxLegal / kW; c++) {
            const int slot = l + kW * c;
            valid[c] = grp_ballot(slot < n && (!allowed || allowed[r * kMaxLegal + slot] != 0), lane);
        }
        candidate_row(keep, valid, priors + r * kMaxLegal, k, reserve, lane, live ? cand + r * k : nullptr);
    }
}

// candidate_row from given masks (qualifies, valid: [B][256] uint8), one
// lane group per root.
__global__ __launch_bounds__(64) void k_candidate_rows(const uint8_t* __restrict__ qual,
                                                       const uint8_t* __restrict__ valid,
                                                       const float* __restrict__ priors, int64_t B, int k,
                                                       int reserve, int32_t* __restrict__ cand) {
    bool live;
    const int64_t r = item_of(B, live);
    const int lane = threadIdx.x, l = gl(lane);
    uint32_t keep[kMaxLegal / kW], ok[kMaxLegal / kW];
#pragma unroll
    for (int c = 0; c < kMaxLegal / kW; c++) {
        keep[c] = grp_ballot(qual[r * kMaxLegal + l + kW * c] != 0, lane);
        ok[c] = grp_ballot(valid[r * kMaxLegal + l + kW * c] != 0, lane);
    }
    candidate_row(keep, ok, priors + r * kMaxLegal, k, reserve, lane, live ? cand + r * k : nullptr);
}

// Philox4x32-10 (Salmon et al., SC'11), first output word.
__device__ __forceinline__ uint32_t philox_word0(uint32_t k0, uint32_t k1, uint32_t c0, uint32_t c1) {
    uint32_t x0 = c0, x1 = c1, x2 = 0, x3 = 0;
#pragma unroll
    for (int r = 0; r < 10; r++) {
        uint32_t hi0 = __umulhi(0xD2511F53u, x0), lo0 = 0xD2511F53u * x0;
        uint32_t hi1 = __umulhi(0xCD9E8D57u, x2), lo1 = 0xCD9E8D57u * x2;
        uint32_t y0 = hi1 ^ x1 ^ k0, y2 = hi0 ^ x3 ^ k1;
        x0 = y0; x1 = lo1; x2 = y2; x3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return x0;
}

// One ply of seeded random play: game i is active while ply < its target
// (philox(seed, (i,0))[0] mod (max_ply+1), or max_ply in lockstep mode) and
// its result is 0; an active game applies legal[(philox(seed,(i,ply+1))[0] *
// n) >> 32].  plies_done[i] counts applied plies.
__global__ void k_random_play_step(uint8_t* __restrict__ states, const uint8_t* __restrict__ moves,
                                   const int32_t* __restrict__ num_legal, int64_t B, int ply, int max_ply,
                                   int lockstep, uint32_t seed, int32_t* __restrict__ plies_done) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B) return;
    uint8_t* s = states + i * kStateBytes;
    int target = lockstep ? max_ply : (int)(philox_word0(seed, 0, (uint32_t)i, 0) % (uint32_t)(max_ply + 1));
    if (ply >= target || s[OFF_RESULT] != 0) return;
    int n = num_legal[i];
    uint32_t u = philox_word0(seed, 0, (uint32_t)i, (uint32_t)(ply + 1));
    int pick = (int)(((uint64_t)u * (uint64_t)n) >> 32);
    const uint8_t* m = moves + (i * kMaxLegal + pick) * 6;
    RowView v{s};
    v.apply(m[0], m[1], m[2] | (m[3] << 8), m[4] | (m[5] << 8));
    if (plies_done) plies_done[i] += 1;
}

// Seeded random play for all its plies in one launch (k_random_play_step
// with its per-ply k_legal<moves>, fused): a workgroup keeps its two games
// (lane groups of 32) from their first ply to their last, the grid striding
// over the games (sized to the workgroups the device holds at once).  A
// game's board is loaded into LDS once and stays there: per ply the group
// rebuilds the derived tables (occupied list, slide exits, articulation
// points), generates the legal list's tables, and one lane decodes the
// Philox-chosen slot (list_slot; the list itself is never written out) and
// applies it to the LDS board, writing the bytes that changed into the
// game's state row (apply_mirrored).  The workgroup moves on when both
// games have stopped (ply >= target or a result): games run for different
// numbers of plies, so after its first pair a workgroup takes the next
// unstarted pair from a device counter (*pair_ctr, zero at launch; one
// atomic per pair), and the grid ends together instead of with the
// workgroups that were dealt a second pair.  Same choices, same rows and
// counts as the per-ply launches, whichever workgroup plays a game.
// Register budget: 5 waves per SIMD (96 VGPRs); at 6 the spills cost more
// than the extra wave.
__global__ void k_zero_u32(uint32_t* __restrict__ p) { *p = 0u; }
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(5))) void k_random_play(
    uint8_t* __restrict__ states, int64_t B, int max_ply, int lockstep, uint32_t seed,
    int32_t* __restrict__ plies_done, uint32_t* __restrict__ pair_ctr) {
    __shared__ Pos PS[kPosPerWave];
    __shared__ int64_t next_first;
    const int grp = threadIdx.x >> 5, l = threadIdx.x & 31;
    Pos& P = PS[grp];
    for (int64_t first = (int64_t)blockIdx.x * kPosPerWave; first < B;) {
        const int64_t i = first + grp;
        const bool live = i < B;
        const int64_t g = live ? i : B - 1;  // a group past the end mirrors the last game and writes nothing
        uint8_t* row = states + g * kStateBytes;
        const int target =
            lockstep ? max_ply : (int)(philox_word0(seed, 0, (uint32_t)g, 0) % (uint32_t)(max_ply + 1));
        int done = 0;
        int result = row[OFF_RESULT];
        bool loaded = false;  // uniform over the workgroup (one wave)
        for (int ply = 0; ply < max_ply; ply++) {
            const bool act = live && ply < target && result == 0;
            if (__ballot(act) == 0ull) break;  // both games of the workgroup have stopped
            if (!loaded) {
                load_position(P, row, threadIdx.x);
                __syncthreads();
                loaded = true;
            }
            prepare_loaded(P, threadIdx.x);
            const ListInfo L = generate_legal(P, threadIdx.x);
            __syncthreads();  // the list's tables before one lane decodes a slot
            if (act && l == 0) {
                const uint32_t u = philox_word0(seed, 0, (uint32_t)g, (uint32_t)(ply + 1));
                const int pick = (int)(((uint64_t)u * (uint64_t)L.n) >> 32);
                int tp = MV_PASS, from = 0, to = 0, seg;
                if (L.total > 0) list_slot(P, L, pick, tp, from, to, seg);
                apply_mirrored(P, row, tp & 0xFF, tp >> 8, from, to);
                done++;
            }
            __syncthreads();  // the board after the move before the next ply reads it
            result = P.result;
        }
        if (live && l == 0 && plies_done) plies_done[g] += done;
        __syncthreads();  // the board's last reads before the next games load
        // the next pair: the grid's first pairs were dealt by block index
        if (threadIdx.x == 0) next_first = ((int64_t)gridDim.x + (int64_t)atomicAdd(pair_ctr, 1u)) * kPosPerWave;
        __syncthreads();
        first = next_first;
    }
}

// legal_mask_kernel (state_encoder.cuh:908-976): the [B][85834] float mask is
// zero-filled (16-byte stores over the whole buffer), then 1.0 is scattered
// at each legal slot's action index (k_legal's fused action output).
constexpr int kActionSpace = 85834;

__global__ void k_zero_f32(float* __restrict__ p, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n4 = count / 4;
    if (i < n4) reinterpret_cast<float4*>(p)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < count - 4 * n4) p[4 * n4 + i] = 0.0f;
}

__global__ void k_mask_scatter(const int32_t* __restrict__ actions, const int32_t* __restrict__ num_legal, int64_t B,
                               float* __restrict__ masks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * kMaxLegal) return;
    const int64_t b = i / kMaxLegal;
    const int slot = (int)(i % kMaxLegal);
    const int a = actions[i];
    if (slot < num_legal[b] && a >= 0 && a < kActionSpace) masks[b * kActionSpace + a] = 1.0f;
}

// ---------------------------------------------------------------- successor rows
// The successor rows of a batch of leaves without a host round trip: the row
// count stays on the device.  k_rows_offsets: exclusive prefix of the
// clamped legal counts (one workgroup, chunks of 4,096 with a running carry)
// and the total; k_rows_map: row -> (leaf, slot); k_successor_rows: the
// successor features of rows < total, kSuccRows per lane group, the grid
// striding over the rows (sized from the capacity, the count read on the
// device).
__global__ __launch_bounds__(1024) void k_rows_offsets(const int32_t* __restrict__ nlegal, int64_t T,
                                                        int64_t* __restrict__ offsets, int64_t* __restrict__ total) {
    // chunks of 4,096 counts, four consecutive counts per thread, with a
    // running carry between chunks
    __shared__ int wsum[16];
    __shared__ int64_t carry_s;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (tid == 0) carry_s = 0;
    __syncthreads();
    for (int64_t base = 0; base < T; base += 4096) {
        int v[4];
        int sum = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int64_t t = base + 4 * tid + j;
            int n = t < T ? nlegal[t] : 0;
            v[j] = n < 0 ? 0 : (n > kMaxLegal ? kMaxLegal : n);
            sum += v[j];
        }
        const int incl = wave_incl_scan(sum);  // at most 64 * 4 * 256 per wave
        if (lane == 63) wsum[w] = incl;
        __syncthreads();
        int64_t run = carry_s + incl - sum;
        for (int k = 0; k < w; k++) run += wsum[k];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int64_t t = base + 4 * tid + j;
            if (t < T) offsets[t] = run;
            run += v[j];
        }
        __syncthreads();
        if (tid == 1023) carry_s = run;
        __syncthreads();
    }
    if (tid == 0) *total = carry_s;
}

__global__ void k_rows_map(const int32_t* __restrict__ nlegal, const int64_t* __restrict__ offsets, int64_t T,
                           int64_t* __restrict__ a2r, int64_t* __restrict__ mi) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T * kMaxLegal) return;
    const int64_t t = i / kMaxLegal;
    const int k = (int)(i % kMaxLegal);
    int n = nlegal[t];
    n = n < 0 ? 0 : (n > kMaxLegal ? kMaxLegal : n);
    if (k < n) {
        a2r[offsets[t] + k] = t;
        mi[offsets[t] + k] = k;
    }
}

// k_rows_plan: the offsets, total and map of k_rows_offsets + k_rows_map in
// one launch, for batches of at most kPlanLeaves leaves (rows_plan_block,
// hive_leaf.hpp).
__global__ __launch_bounds__(256) void k_rows_plan(const int32_t* __restrict__ nlegal, int64_t T,
                                                   int64_t* __restrict__ offsets, int64_t* __restrict__ total,
                                                   int64_t* __restrict__ a2r, int64_t* __restrict__ mi) {
    rows_plan_block(nlegal, T, offsets, total, a2r, mi, (int)blockIdx.x);
}

template <typename Ix>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(kSuccWaves<Ix>))) void k_successor_rows(const uint8_t* __restrict__ states,
                                                       const uint8_t* __restrict__ legal,
                                                       const int64_t* __restrict__ a2r,
                                                       const int64_t* __restrict__ midx,
                                                       const int64_t* __restrict__ total, int64_t num_roots,
                                                       float* __restrict__ feat_out) {
    successor_stream<Ix>(states, legal, a2r, midx, (Ix)*total, num_roots, feat_out);
}

inline int grid_for(int64_t n, int block) { return (int)((n + block - 1) / block); }

inline int finish() { return (int)hipGetLastError(); }

}  // namespace

// ============================================================== C-ABI
extern "C" {

int hg_abi_version(void) { return HG_ABI_VERSION; }

// The geometry is closed-form (no tables to upload); set-up looks up the current
// device's scratch array of the no-allocation probe entry point.
int hg_initialize_tables(void) { return hg_probe_scratch_init(); }

int hg_create_initial_states(uint8_t* states, int64_t B, int expansion_mask, void* stream) {
    if (B <= 0) return 0;
    int64_t chunks = B * (kStateBytes / 16);
    hipLaunchKernelGGL(k_init_states, dim3(grid_for(chunks, 256)), dim3(256), 0, (hipStream_t)stream,
                       reinterpret_cast<uint4*>(states), chunks, expansion_mask);
    return finish();
}

int hg_apply_moves(uint8_t* states, const uint8_t* moves, int64_t B, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(k_apply_moves, dim3(grid_for(B, 256)), dim3(256), 0, (hipStream_t)stream, states, moves, B);
    return finish();
}

int hg_check_results(const uint8_t* states, int64_t B, int32_t* results, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(k_check_results, dim3(grid_for(B, 256)), dim3(256), 0, (hipStream_t)stream, states, B,
                       results);
    return finish();
}

int hg_generate_legal_moves(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* num_legal, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL((k_legal<true, false, false>), dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, (hipStream_t)stream, states, B,
                       moves, num_legal, nullptr, nullptr);
    return finish();
}

int hg_generate_legal_moves_and_fnn_features(const uint8_t* states, int64_t B, uint8_t* moves,
                                             int32_t* num_legal, float* features, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL((k_legal<true, true, false>), dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, (hipStream_t)stream, states, B,
                       moves, num_legal, features, nullptr);
    return finish();
}

int hg_legal_features_actions(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* num_legal,
                              float* features, int32_t* actions, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL((k_legal<true, true, true>), dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, (hipStream_t)stream, states, B,
                       moves, num_legal, features, actions);
    return finish();
}

int64_t hg_legal_features_actions_ordered_workspace(int64_t B) {
    return B <= 0 ? 0 : (int64_t)sizeof(int32_t) * (2 * kOrderBuckets + kOrderBuckets * B);
}

int hg_legal_features_actions_ordered(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* num_legal,
                                      float* features, int32_t* actions, void* workspace, int parity,
                                      void* stream) {
    if (B <= 0) return 0;
    if (!workspace || (parity & ~1) || B > INT32_MAX) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    int32_t* counts = reinterpret_cast<int32_t*>(workspace) + parity * kOrderBuckets;
    int32_t* clear = reinterpret_cast<int32_t*>(workspace) + (parity ^ 1) * kOrderBuckets;
    int32_t* lists = reinterpret_cast<int32_t*>(workspace) + 2 * kOrderBuckets;
    hipLaunchKernelGGL(k_order_buckets, dim3((unsigned)grid_for(B, kOrderPer)), dim3(256), 0, s, states, B, counts,
                       clear, lists);
    hipLaunchKernelGGL((k_legal<true, true, true, true>), dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, s,
                       states, B, moves, num_legal, features, actions, counts, lists);
    return finish();
}

int hg_legal_mask(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* num_legal, int32_t* actions,
                  float* masks, void* stream) {
    if (B <= 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL((k_legal<true, false, true>), dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, s, states, B,
                       moves, num_legal, nullptr, actions);
    const int64_t count = B * (int64_t)kActionSpace;
    hipLaunchKernelGGL(k_zero_f32, dim3((unsigned)((count / 4 + 255) / 256)), dim3(256), 0, s, masks, count);
    hipLaunchKernelGGL(k_mask_scatter, dim3((unsigned)((B * kMaxLegal + 255) / 256)), dim3(256), 0, s, actions,
                       num_legal, B, masks);
    return finish();
}

int hg_extract_fnn_features(const uint8_t* states, const uint8_t* moves, const int32_t* num_legal, int64_t B,
                            float* features, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(k_extract_features, dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, (hipStream_t)stream, states, moves,
                       num_legal, B, features);
    return finish();
}

int hg_legal_moves_to_actions(const uint8_t* states, const uint8_t* moves, const int32_t* num_legal, int64_t B,
                              int32_t* actions, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(k_actions, dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, (hipStream_t)stream, states, moves, num_legal, B,
                       actions, (int32_t*)nullptr);
    return finish();
}

int hg_compute_centroids(const uint8_t* states, int64_t B, int32_t* centroids, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(k_actions, dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, (hipStream_t)stream, states,
                       (const uint8_t*)nullptr, (const int32_t*)nullptr, B, (int32_t*)nullptr, centroids);
    return finish();
}

int64_t hg_successor_rows_workspace(int64_t T) { return T <= 0 ? 0 : 8 * (T + 1 + 2 * T * (int64_t)kMaxLegal); }

int hg_successor_rows(const uint8_t* states, const uint8_t* legal_moves, const int32_t* num_legal, int64_t T,
                      void* workspace, float* features, void* stream) {
    if (T <= 0) return 0;
    if (((uintptr_t)workspace & 7)) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    if (T <= kPlanLeaves) {
        const RowsPlan R = rows_plan_of(workspace, T);
        hipLaunchKernelGGL(k_rows_plan, dim3((unsigned)((T + 255) / 256)), dim3(256), 0, s, num_legal, T, R.offsets,
                           R.total, R.a2r, R.mi);
    } else {
        int e = successor_rows_plan_large(num_legal, T, workspace, s);
        if (e) return e;
    }
    return successor_rows_after_plan(states, legal_moves, T, workspace, features, s);
}

int hg_fnn_successor_features(const uint8_t* states, const uint8_t* legal_moves, int64_t num_roots,
                              const int64_t* action_to_root, const int64_t* move_indices, int64_t N, float* features,
                              void* stream) {
    if (N <= 0) return 0;
    const int64_t pairs = (N + kSuccRows * kPosPerWave - 1) / (kSuccRows * kPosPerWave);
    const dim3 grid((unsigned)(pairs < kSuccGrid ? pairs : kSuccGrid));
    if (successor_narrow(N, num_roots))
        hipLaunchKernelGGL(k_successor_features<uint32_t>, grid, dim3(64), 0, (hipStream_t)stream, states, legal_moves,
                           action_to_root, move_indices, N, num_roots, features);
    else
        hipLaunchKernelGGL(k_successor_features<int64_t>, grid, dim3(64), 0, (hipStream_t)stream, states, legal_moves,
                           action_to_root, move_indices, N, num_roots, features);
    return finish();
}

int hg_reserve_candidates(const uint8_t* states, const uint8_t* legal_moves, const int32_t* num_legal,
                          const uint8_t* allowed, const float* priors, int64_t B, int k, int reserve,
                          int immobile_only, uint8_t* qualifies, int32_t* candidates, void* stream) {
    if (B <= 0) return 0;
    if (candidates && (!priors || k < 1 || k > kMaxLegal || reserve < 0 || reserve > k))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_reserve_qualify, dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, (hipStream_t)stream,
                       states, legal_moves, num_legal, B, immobile_only, qualifies, allowed, priors, k, reserve,
                       candidates);
    return finish();
}

int hg_candidate_rows(const uint8_t* qualifies, const uint8_t* valid, const float* priors, int64_t B, int k,
                      int reserve, int32_t* candidates, void* stream) {
    if (B <= 0) return 0;
    if (k < 1 || k > kMaxLegal || reserve < 0 || reserve > k) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_candidate_rows, dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, (hipStream_t)stream,
                       qualifies, valid, priors, B, k, reserve, candidates);
    return finish();
}

int hg_queen_escape_flags(const uint8_t* states, int64_t B, uint8_t* flags, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(k_queen_escape, dim3((unsigned)grid_for(B, kPosPerWave)), dim3(64), 0, (hipStream_t)stream, states, B, flags);
    return finish();
}

int hg_random_play(uint8_t* states, uint8_t* moves, int64_t B, int max_ply, int lockstep, uint32_t seed,
                   int32_t* plies_done, void* stream) {
    if (B <= 0 || max_ply <= 0) return 0;
    if (!moves || B > INT32_MAX) return (int)hipErrorInvalidValue;
    int dev = 0, cus = 0, per_cu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_random_play, 64, 0);
    if (e != hipSuccess) return (int)e;
    const int64_t pairs = (B + kPosPerWave - 1) / kPosPerWave;
    const int64_t resident = (int64_t)(cus > 0 ? cus : 1) * (per_cu > 0 ? per_cu : 1);
    // the pair counter in the scratch (its first 4-byte aligned word; the
    // scratch holds at least 1,536 bytes), zeroed by a kernel
    uint32_t* ctr = reinterpret_cast<uint32_t*>(((uintptr_t)moves + 3) & ~(uintptr_t)3);
    hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(1), 0, (hipStream_t)stream, ctr);
    hipLaunchKernelGGL(k_random_play, dim3((unsigned)(pairs < resident ? pairs : resident)), dim3(64), 0,
                       (hipStream_t)stream, states, B, max_ply, lockstep, seed, plies_done, ctr);
    return finish();
}

int hg_random_play_step(uint8_t* states, const uint8_t* moves, const int32_t* num_legal, int64_t B, int ply,
                        int max_ply, int lockstep, uint32_t seed, int32_t* plies_done, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(k_random_play_step, dim3(grid_for(B, 256)), dim3(256), 0, (hipStream_t)stream, states, moves,
                       num_legal, B, ply, max_ply, lockstep, seed, plies_done);
    return finish();
}

}  // extern "C"

namespace hw {

int successor_rows_plan_large(const int32_t* num_legal, int64_t T, void* workspace, hipStream_t s) {
    const RowsPlan R = rows_plan_of(workspace, T);
    hipLaunchKernelGGL(k_rows_offsets, dim3(1), dim3(1024), 0, s, num_legal, T, R.offsets, R.total);
    hipLaunchKernelGGL(k_rows_map, dim3((unsigned)((T * kMaxLegal + 255) / 256)), dim3(256), 0, s, num_legal,
                       R.offsets, T, R.a2r, R.mi);
    return finish();
}

int successor_rows_after_plan(const uint8_t* states, const uint8_t* legal_moves, int64_t T, void* workspace,
                              float* features, hipStream_t s) {
    const RowsPlan R = rows_plan_of(workspace, T);
    const int64_t pairs = (T * kMaxLegal + kSuccRows * kPosPerWave - 1) / (kSuccRows * kPosPerWave);
    const unsigned grid = (unsigned)(pairs < kSuccGrid ? pairs : kSuccGrid);
    if (successor_narrow(T * kMaxLegal, T))  // at most 256 rows per leaf
        hipLaunchKernelGGL(k_successor_rows<uint32_t>, dim3(grid), dim3(64), 0, s, states, legal_moves, R.a2r, R.mi,
                           R.total, T, features);
    else
        hipLaunchKernelGGL(k_successor_rows<int64_t>, dim3(grid), dim3(64), 0, s, states, legal_moves, R.a2r, R.mi,
                           R.total, T, features);
    return finish();
}

}  // namespace hw
