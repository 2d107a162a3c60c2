// hive_probe.hip -- root_tactical_probe_batch (game_logic.cu:1579-1616 over
// root_tactical_probe_kernel :290-397) as six launches on the caller's
// stream, no host synchronisation:
//
//   k_probe_roots   one lane group per root (hive_probe.hpp probe_root):
//                   allowed[] = legal slots, the immediate win, the gates of
//                   the screen and two-move stages (kept in forced[] until
//                   k_probe_finish), and the (root, move) jobs of both
//                   stages appended to the workspace's job lists;
//   k_probe_jobs    one lane group per screen job: allowed[r][i] = 0 when
//                   the opponent wins at once after move i; and, in the same
//                   launch, one lane group per two-move candidate:
//                   fail[candidate] = 1 when a reply lowers the opponent
//                   queen's surround, else the candidate's grandchildren
//                   (its replies that do not already win for the root
//                   player) go to the grandchild list; a candidate whose
//                   grandchildren do not fit is appended to the overflow
//                   list;
//   k_probe_grand   one lane group per listed grandchild of an allowed
//                   candidate: fail[candidate] = 1 when the root player does
//                   not win at once; and, in the same launch, one lane group
//                   per (overflow candidate, part): the part's
//                   grandchildren, fail[candidate] = 1 when one is not won;
//   k_probe_win2_commit  per candidate no stage failed: the lowest passing
//                   slot of each root by atomic min (winning[] holds
//                   kUndecided meanwhile);
//   k_probe_finish  per root: kUndecided -> -1, forced = the screen ran and
//                   left no move allowed.
//
// The job kernels stride over their lists with a grid sized from the batch;
// the list lengths are read on the device.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/hive_gpu.h"
#include "hive_probe.hpp"

using namespace hw;

namespace {

constexpr int64_t kUndecided = 1 << 20;  // above every slot; replaced by -1 at the end
constexpr int kJobGrid = 4096;           // workgroups of the job kernels (two jobs each per pass)

// counters[0]: screen jobs, [1]: two-move candidates, [2]: overflow
// candidates, [4..5]: grandchild-list reservations, 64-bit (may pass the
// capacity); [3], [6], [7] unused (the lists start 32 bytes in)
constexpr int kCounters = 8;
__device__ __forceinline__ unsigned long long* reservations(int32_t* counters) {
    return reinterpret_cast<unsigned long long*>(counters + 4);
}
__global__ void k_probe_reset(int32_t* __restrict__ counters) {
    if (threadIdx.x < kCounters) counters[threadIdx.x] = 0;
}

__global__ __launch_bounds__(64) void k_probe_roots(const uint8_t* __restrict__ states,
                                                    const uint8_t* __restrict__ legal,
                                                    const int32_t* __restrict__ num_legal,
                                                    const float* __restrict__ priors, int64_t B, int win1, int screen,
                                                    int win2, int64_t* __restrict__ winning,
                                                    uint8_t* __restrict__ allowed, uint8_t* __restrict__ gate_out,
                                                    int32_t* __restrict__ counters, int32_t* __restrict__ jobs_screen,
                                                    int32_t* __restrict__ jobs_win2, int32_t* __restrict__ fail_win2) {
    __shared__ Pos PS[kPosPerWave];
    const int lane = threadIdx.x, l = gl(lane);
    const int64_t r0 = (int64_t)blockIdx.x * kPosPerWave + (lane >> 5);
    const bool live = r0 < B;
    const int64_t r = live ? r0 : B - 1;
    RootProbe R = probe_root(PS[lane >> 5], states + r * kStateBytes, legal + r * (kMaxLegal * 6), num_legal[r],
                             priors + r * kMaxLegal, win1 != 0, screen != 0, win2 != 0, lane);
    if (!live) return;
    for (int i = l; i < kMaxLegal; i += kW) allowed[r * kMaxLegal + i] = i < R.n ? 1 : 0;
    if (l == 0) {
        winning[r] = R.win >= 0 ? R.win : ((R.gate & kProbeWin2) ? kUndecided : -1);
        gate_out[r] = (uint8_t)R.gate;
    }
    if (R.gate & kProbeScreen) {
        int base = 0;
        if (l == 0) base = atomicAdd(&counters[0], R.n);
        base = grp_shfl(base, 0, lane);
        for (int i = l; i < R.n; i += kW) jobs_screen[base + i] = (int32_t)(r * kMaxLegal + i);
    }
    if (R.gate & kProbeWin2) {
        int nc = 0;
        for (int k = 0; k < 8; k++) nc += __popc(R.cand[k]);
        int base = 0;
        if (l == 0 && nc) base = atomicAdd(&counters[1], nc);
        base = grp_shfl(base, 0, lane);
        if (l == 0) {
            int j = base;
            for (int k = 0; k < 8; k++)
                for (uint32_t w = R.cand[k]; w; w &= w - 1) {
                    fail_win2[j] = 0;
                    jobs_win2[j++] = (int32_t)(r * kMaxLegal + 32 * k + __ffs(w) - 1);
                }
        }
    }
}

// The screen jobs and the two-move candidates' drop stage in one launch:
// the two are independent (the drop stage lists the grandchildren of every
// candidate, and the later stages skip the candidates the screen
// disallows).  Waves [0, w_screen) take pairs of screen jobs, the rest pairs
// of candidates; the branch is uniform per wave.
__global__ __launch_bounds__(64) void k_probe_jobs(const uint8_t* __restrict__ states,
                                                   const uint8_t* __restrict__ legal,
                                                   int32_t* __restrict__ counters,
                                                   const int32_t* __restrict__ jobs_screen,
                                                   const int32_t* __restrict__ jobs_win2,
                                                   uint8_t* __restrict__ allowed, int32_t* __restrict__ fail,
                                                   int32_t* __restrict__ overflow, int32_t* __restrict__ gc,
                                                   int64_t cap) {
    __shared__ Pos PS[kPosPerWave];
    const int lane = threadIdx.x;
    const int64_t n_screen = counters[0], n_cand = counters[1];
    const int64_t w_screen = (n_screen + 1) / 2, w_total = w_screen + (n_cand + 1) / 2;
    for (int64_t p = blockIdx.x; p < w_total; p += gridDim.x) {  // uniform over the workgroup
        if (p < w_screen) {
            const int64_t j0 = 2 * p + (lane >> 5);
            const bool live = j0 < n_screen;
            const int job = jobs_screen[live ? j0 : 2 * p];
            const int64_t r = job / kMaxLegal, i = job % kMaxLegal;
            const bool bad =
                probe_screen(PS[lane >> 5], states + r * kStateBytes, legal + (r * kMaxLegal + i) * 6, lane);
            if (live && gl(lane) == 0) allowed[job] = bad ? 0 : 1;
        } else {
            const int64_t q = p - w_screen;
            const int64_t j0 = 2 * q + (lane >> 5);
            const bool live = j0 < n_cand;
            const int64_t j = live ? j0 : 2 * q;
            const int job = jobs_win2[j];
            const int64_t r = job / kMaxLegal, i = job % kMaxLegal;
            const int res = probe_drop_list(PS[lane >> 5], states + r * kStateBytes,
                                            legal + (r * kMaxLegal + i) * 6, live, (int32_t)j,
                                            reservations(counters), gc, cap, lane);
            if (live && gl(lane) == 0) {
                if (res == kDropped) fail[j] = 1;
                else if (res == kOverflow) overflow[atomicAdd(&counters[2], 1)] = (int32_t)j;
            }
        }
        __syncthreads();
    }
}

// The listed grandchildren and the overflow candidates' part programs in one
// launch: waves [0, w_grand) take pairs of grandchild entries, the rest pairs
// of (overflow candidate, part); the branch is uniform per wave.  A
// candidate the screen disallowed, or one already failed, is skipped.
__global__ __launch_bounds__(64) void k_probe_grand(const uint8_t* __restrict__ states,
                                                    const uint8_t* __restrict__ legal,
                                                    int32_t* __restrict__ counters,
                                                    const int32_t* __restrict__ jobs,
                                                    const uint8_t* __restrict__ allowed,
                                                    const int32_t* __restrict__ gc, int64_t cap,
                                                    const int32_t* __restrict__ overflow,
                                                    int32_t* __restrict__ fail) {
    __shared__ Pos PS[kPosPerWave];
    __shared__ Replies RS[kPosPerWave];
    const int lane = threadIdx.x;
    const int64_t reserved = (int64_t)*reservations(counters);
    const int64_t n_grand = reserved < cap ? reserved : cap;
    const int64_t n_parts = (int64_t)counters[2] * kWin2Parts;  // (overflow candidate, part)
    const int64_t w_grand = (n_grand + 1) / 2, w_total = w_grand + (n_parts + 1) / 2;
    for (int64_t p = blockIdx.x; p < w_total; p += gridDim.x) {  // uniform over the workgroup
        if (p < w_grand) {
            const int64_t g0 = 2 * p + (lane >> 5);
            const bool live = g0 < n_grand;
            const int64_t g = live ? g0 : 2 * p;
            const int32_t j = gc[2 * g];
            const int job = jobs[j >= 0 ? j : 0];  // jobs[0] exists whenever an entry does
            // a sentinel entry (-1), a disallowed candidate or one already failed
            const bool active = live && j >= 0 && allowed[job] != 0 && fail[j] == 0;
            if (!hw_wave_any(active)) continue;  // uniform: one wave per workgroup
            const int64_t r = job / kMaxLegal, i = job % kMaxLegal;
            const bool won = probe_grand(PS[lane >> 5], states + r * kStateBytes,
                                         legal + (r * kMaxLegal + i) * 6, (uint32_t)gc[2 * g + 1], lane);
            if (active && !won && gl(lane) == 0) fail[j] = 1;
        } else {
            const int64_t q0 = 2 * (p - w_grand) + (lane >> 5);
            const bool live = q0 < n_parts;
            const int64_t q = live ? q0 : 2 * (p - w_grand);
            const int64_t j = overflow[q / kWin2Parts];
            const int job = jobs[j];
            const int64_t r = job / kMaxLegal, i = job % kMaxLegal;
            const bool active = live && allowed[job] != 0;
            const bool ok = probe_win2(PS[lane >> 5], RS[lane >> 5], states + r * kStateBytes,
                                       legal + (r * kMaxLegal + i) * 6, active, (int)(q % kWin2Parts), lane);
            if (active && !ok && gl(lane) == 0) fail[j] = 1;
        }
        __syncthreads();
    }
}

// a candidate no stage failed wins: the lowest such slot of each root
__global__ void k_probe_win2_commit(const int32_t* __restrict__ counters, const int32_t* __restrict__ jobs,
                                    const uint8_t* __restrict__ allowed, const int32_t* __restrict__ fail,
                                    int64_t* __restrict__ winning) {
    const int64_t count = counters[1];
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < count; j += (int64_t)gridDim.x * blockDim.x) {
        const int job = jobs[j];
        if (allowed[job] != 0 && fail[j] == 0)
            atomicMin(reinterpret_cast<unsigned long long*>(winning + job / kMaxLegal), (unsigned long long)(job % kMaxLegal));
    }
}

__global__ void k_probe_finish(const int32_t* __restrict__ num_legal, int64_t B, int64_t* __restrict__ winning,
                               const uint8_t* __restrict__ allowed, uint8_t* __restrict__ forced) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= B) return;
    if (winning[r] == kUndecided) winning[r] = -1;
    const int gate = forced[r];
    uint8_t f = 0;
    if (gate & kProbeScreen) {
        int n = num_legal[r];
        n = n < 0 ? 0 : (n > kMaxLegal ? kMaxLegal : n);
        bool any = false;
        for (int i = 0; i < n; i++) any |= allowed[r * kMaxLegal + i] != 0;
        f = any ? 0 : 1;
    }
    forced[r] = f;
}

// Scratch of the no-allocation entry point: the probe's job counters, job
// lists, failure flags and grandchild list for up to HG_PROBE_NOALLOC_MAX_ROOTS
// roots (25.2 MB), one copy per GPU, held until the process ends.  Host code never
// uses the symbol itself (on the host it names a stand-in, not device
// memory): it uses the per-device address hipGetSymbolAddress returns.
// counters, then four lists of B * 256 int32 (screen jobs, two-move
// candidates, their failure flags, overflow candidates) and the grandchild
// list of B * 256 pairs
constexpr int64_t kListInts = 6;
constexpr int64_t kScratchInts = kCounters + kListInts * (int64_t)HG_PROBE_NOALLOC_MAX_ROOTS * kMaxLegal;
__device__ __align__(256) int32_t scratch[kScratchInts];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch[kMaxDevices] = {};

// The current device's scratch address: looked up on the device's first use
// and kept; `refresh` looks it up again (after a device reset the old address
// is stale).
int scratch_of_current_device(int32_t** out, bool refresh) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (refresh || g_scratch[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        g_scratch[dev] = static_cast<int32_t*>(p);
    }
    *out = g_scratch[dev];
    return 0;
}

}  // namespace

extern "C" {

int hg_probe_scratch_init(void) {
    int32_t* p = nullptr;
    return scratch_of_current_device(&p, true);
}

int64_t hg_root_tactical_probe_workspace(int64_t B) { return B <= 0 ? 0 : kCounters + kListInts * B * kMaxLegal; }

int hg_root_tactical_probe(const uint8_t* states, const uint8_t* legal_moves, const int32_t* num_legal,
                           const float* priors, int64_t B, int enable_win_in_one, int enable_check_opponent_wins,
                           int enable_win_in_two, int64_t* winning, uint8_t* allowed, uint8_t* forced,
                           int32_t* workspace, void* stream) {
    if (B <= 0) return 0;
    if (B > (int64_t)(INT32_MAX / kMaxLegal)) return (int)hipErrorInvalidValue;
    // the grandchild-list counter is a 64-bit atomic at counters + 4
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 7u)) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    int32_t* counters = workspace;
    int32_t* jobs_screen = workspace + kCounters;
    int32_t* jobs_win2 = jobs_screen + B * kMaxLegal;
    int32_t* fail_win2 = jobs_win2 + B * kMaxLegal;
    int32_t* overflow = fail_win2 + B * kMaxLegal;
    int32_t* gc = overflow + B * kMaxLegal;  // (candidate, packed reply) pairs
    const int64_t cap = B * kMaxLegal;
    hipLaunchKernelGGL(k_probe_reset, dim3(1), dim3(64), 0, s, counters);
    hipLaunchKernelGGL(k_probe_roots, dim3((unsigned)((B + kPosPerWave - 1) / kPosPerWave)), dim3(64), 0, s, states,
                       legal_moves, num_legal, priors, B, enable_win_in_one, enable_check_opponent_wins,
                       enable_win_in_two, winning, allowed, forced, counters, jobs_screen, jobs_win2, fail_win2);
    const int64_t pairs = B * kMaxLegal;  // screen jobs and candidates: at most B * 256 each
    const unsigned grid = (unsigned)(pairs < kJobGrid ? pairs : kJobGrid);
    hipLaunchKernelGGL(k_probe_jobs, dim3(grid), dim3(64), 0, s, states, legal_moves, counters, jobs_screen,
                       jobs_win2, allowed, fail_win2, overflow, gc, cap);
    hipLaunchKernelGGL(k_probe_grand, dim3((unsigned)kJobGrid), dim3(64), 0, s, states, legal_moves, counters,
                       jobs_win2, allowed, gc, cap, overflow, fail_win2);
    hipLaunchKernelGGL(k_probe_win2_commit, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, s, counters, jobs_win2,
                       allowed, fail_win2, winning);
    hipLaunchKernelGGL(k_probe_finish, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, s, num_legal, B, winning,
                       allowed, forced);
    return (int)hipGetLastError();
}

int hg_root_tactical_probe_noalloc(const uint8_t* states, const uint8_t* legal_moves, const int32_t* num_legal,
                                   const float* priors, int64_t B, int enable_win_in_one,
                                   int enable_check_opponent_wins, int enable_win_in_two, int64_t* winning,
                                   uint8_t* allowed, uint8_t* forced, void* stream) {
    if (B <= 0) return 0;
    if (B > HG_PROBE_NOALLOC_MAX_ROOTS) return (int)hipErrorInvalidValue;
    int32_t* ws = nullptr;
    const int err = scratch_of_current_device(&ws, false);
    if (err != 0) return err;
    return hg_root_tactical_probe(states, legal_moves, num_legal, priors, B, enable_win_in_one,
                                  enable_check_opponent_wins, enable_win_in_two, winning, allowed, forced, ws, stream);
}

}  // extern "C"
