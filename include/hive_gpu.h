/*
 * hive_gpu.h -- C-ABI of libhive_gpu.so, the MI355X (gfx950) batched Hive
 * engine.  This is the drop-in boundary: the Python package
 * hive_neuralnet_amd.hive_gpu (the counterpart of the reference's
 * hive_gpu.load_extension()) binds these symbols with ctypes; any other FFI
 * can bind them the same way.
 *
 * Conventions (all entry points):
 *   - pointers are device pointers; the caller allocates every input and
 *     output (the reference allocates outputs inside its wrappers -- the
 *     Python layer does that here, with the reference's fill values);
 *   - `stream` is a hipStream_t (void* so this header needs no HIP headers);
 *     work is enqueued on it and the call returns without synchronising;
 *   - the return value is a hipError_t code (0 = success) of the launch;
 *   - sizes <= 0 are a no-op returning 0;
 *   - byte formats are the reference's: a state row is 3424 bytes
 *     (HiveState, hive_gpu/csrc/hive_state.cuh:239-269), a move is 6 bytes
 *     {u8 type, u8 piece_type, u16 from, u16 to} (hive_state.cuh:228-233),
 *     legal lists are [B, 256, 6] with zero padding, features are [B, 122].
 *
 * Each declaration names the reference interface it replaces
 * (chrismejias/hive_neuralnet, file:line).
 */
#ifndef HIVE_GPU_H
#define HIVE_GPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HG_ABI_VERSION 1
#define HG_STATE_BYTES 3424
#define HG_MOVE_BYTES 6
#define HG_MAX_LEGAL_MOVES 256
#define HG_FNN_FEAT_DIM 122

int hg_abi_version(void);

/* initialize_tables -- hive_gpu/csrc/game_logic.cu:404-407, bindings.cpp:257.
 * The hex tables are closed-form constants here; kept for API parity. */
int hg_initialize_tables(void);

/* create_initial_states -- game_logic.cu:413-428 (init_states_kernel :54-59).
 * Writes every byte of states[B][3424]. */
int hg_create_initial_states(uint8_t* states, int64_t B, int expansion_mask, void* stream);

/* apply_moves_batch -- game_logic.cu:465-477 (apply_moves_kernel :233-242).
 * moves[B][6]; states updated in place. */
int hg_apply_moves(uint8_t* states, const uint8_t* moves, int64_t B, void* stream);

/* check_results_batch -- game_logic.cu:483-497.  results[B] int32. */
int hg_check_results(const uint8_t* states, int64_t B, int32_t* results, void* stream);

/* generate_legal_moves_batch -- game_logic.cu:436-459.
 * moves[B][256][6] (fully written, zero padded), num_legal[B]. */
int hg_generate_legal_moves(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* num_legal, void* stream);

/* generate_legal_moves_and_fnn_features_batch -- game_logic.cu:1439-1464. */
int hg_generate_legal_moves_and_fnn_features(const uint8_t* states, int64_t B, uint8_t* moves,
                                             int32_t* num_legal, float* features, void* stream);

/* Fused move generation + FNN features + action indices in one pass: the
 * outputs of generate_legal_moves_and_fnn_features_batch (game_logic.cu:1439)
 * followed by legal_moves_to_actions_batch (game_logic.cu:837) without the
 * list round trip through HBM.  actions[B][256] int32, -1 padded.  No single
 * reference entry point; same spirit as the reference's own fused
 * mcts_select_replay_legal_fnn_root_slots_batch. */
int hg_legal_features_actions(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* num_legal,
                              float* features, int32_t* actions, void* stream);

/* hg_legal_features_actions taking the positions in buckets of 4 turns,
 * latest first (a wave's cost is its longer position; the launch ends with
 * its longest waves): identical outputs.  workspace:
 * hg_legal_features_actions_ordered_workspace(B) bytes, 4-byte aligned: two
 * arrays of 32 bucket counts, then one index list per bucket.  A call needs
 * counts[parity] zero, uses it and clears counts[parity ^ 1]: zero-fill a new
 * workspace once, then alternate parity (0, 1, 0, ...) on calls that use it
 * on one stream.  A HIP graph replays the parity it captured and would count
 * into arrays that nothing clears: capture hg_legal_features_actions instead
 * (the Python mirror does so while its stream is capturing).  No reference
 * counterpart (same outputs as the entry above). */
int64_t hg_legal_features_actions_ordered_workspace(int64_t B);
int hg_legal_features_actions_ordered(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* num_legal,
                                      float* features, int32_t* actions, void* workspace, int parity,
                                      void* stream);

/* extract_fnn_features_batch -- game_logic.cu:1409-1431.
 * features for caller-supplied lists (num_legal clamped to [0, 256]). */
int hg_extract_fnn_features(const uint8_t* states, const uint8_t* moves, const int32_t* num_legal, int64_t B,
                            float* features, void* stream);

/* legal_moves_to_actions_batch -- game_logic.cu:837-857.
 * actions[B][256] int32: action index per listed move, -1 beyond num_legal
 * and for moves outside the 17x17 window around the centroid. */
int hg_legal_moves_to_actions(const uint8_t* states, const uint8_t* moves, const int32_t* num_legal, int64_t B,
                              int32_t* actions, void* stream);

/* compute_centroids_batch -- game_logic.cu:910-926.  centroids[B][2] int32. */
int hg_compute_centroids(const uint8_t* states, int64_t B, int32_t* centroids, void* stream);

/* fnn_successor_features_batch -- game_logic.cu:1648-1671.
 * For i < N: features[i] of states[action_to_root[i]] after
 * legal_moves[action_to_root[i]][move_indices[i]], with the compact
 * successor move summary (move_gen.cuh:1416-1563).  num_roots is the row
 * count of states/legal_moves; rows whose root or move index is out of range
 * get all-zero features (the reference reads out of bounds there). */
int hg_fnn_successor_features(const uint8_t* states, const uint8_t* legal_moves, int64_t num_roots,
                              const int64_t* action_to_root, const int64_t* move_indices, int64_t N, float* features,
                              void* stream);

/* hg_fnn_leaf_eval -- FNN leaf evaluation, fused (restates the torch chain of
 * the reference's FNNMCTSOrchestrator._eval_states,
 * hive_fnn/fnn_mcts_orchestrator.py:243-316, over HiveFNN.encode / value_head /
 * score_actions, hive_fnn/fnn_network.py:175-220; the reference has no kernel
 * for it).  Network widths: hidden = embedding = action tower = 64, F <= 128
 * features (even).  Weights are the nn.Linear / nn.LayerNorm tensors as
 * stored (row-major [out][in]).
 *
 * features[T + N][F]: the T leaf rows, then the successor rows; the
 * successor rows of leaf t are T + offsets[t] .. + num_legal[t], and
 * succ_leaf[i] = t for successor row i (i < N).  With
 *   e(x)          = fc2(LayerNorm(sigmoid(fc1 x)))     (eps 1e-5)
 *   root_values[t] = tanh(value_w . e(leaf t) + value_b)
 *   child_q[t][i]  = -tanh(value_w . e(successor i of t) + value_b)
 *   logit_i        = action2_w . sigmoid(action1_w [e(leaf t) | e(succ i)]
 *                                        + action1_b) + action2_b
 *   priors[t][i]   = softmax over i < num_legal[t] of logit_i
 * priors and child_q are [T][256], zero beyond num_legal[t].
 * workspace: T * 64 + 2 * N floats, 16-byte aligned (the root half of the
 * action tower per leaf, then logits and child values per successor row);
 * features must be 8-byte aligned.  Returns hipErrorInvalidValue for other
 * shapes or alignments. */
int hg_fnn_leaf_eval(const float* features, int64_t T, int64_t N, int F, const int64_t* offsets,
                     const int32_t* num_legal, const int64_t* succ_leaf, const float* fc1_w, const float* fc1_b,
                     const float* ln_w, const float* ln_b, const float* fc2_w, const float* fc2_b,
                     const float* value_w, float value_b, const float* action1_w, const float* action1_b,
                     const float* action2_w, float action2_b, float* workspace, float* priors, float* root_values,
                     float* child_q, void* stream);

/* root_tactical_probe_batch -- game_logic.cu:1579-1616 (root_tactical_probe_kernel
 * :290-397; has_immediate_surround_win_for_current_player and
 * generate_non_decreasing_surround_replies, move_gen.cuh:825-898).  For each
 * root: winning[B] int64 = the immediate win with the highest prior (first on
 * ties; only when the opponent's queen has 5 neighbours), else the lowest
 * slot after which every reply loses at once (opponent queen at 4 or 5),
 * else -1; allowed[B][256] uint8 = legal slots, minus those after which the
 * opponent wins at once (only when the own queen has 5 neighbours);
 * forced[B] uint8 = that screen left no slot.  num_legal is clamped to 256.
 * workspace: hg_root_tactical_probe_workspace(B) int32, 8-byte aligned (job
 * counters, job lists, the two-move candidates' failure flags and their
 * grandchildren's list).  Six launches on `stream`, no host
 * synchronisation. */
int64_t hg_root_tactical_probe_workspace(int64_t B);
int hg_root_tactical_probe(const uint8_t* states, const uint8_t* legal_moves, const int32_t* num_legal,
                           const float* priors, int64_t B, int enable_win_in_one, int enable_check_opponent_wins,
                           int enable_win_in_two, int64_t* winning, uint8_t* allowed, uint8_t* forced,
                           int32_t* workspace, void* stream);

/* hg_root_tactical_probe with no workspace argument and no allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The job lists live in a static device array of this
 * library, one per GPU, sized for at most HG_PROBE_NOALLOC_MAX_ROOTS roots
 * (25.2 MB); B above that returns hipErrorInvalidValue and launches nothing.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other streams, other threads) race and must be serialised by the
 * caller (the Python binding orders its own calls on one GPU by an event,
 * outside graph capture).  Outputs as hg_root_tactical_probe.
 * hg_probe_scratch_init looks up the current device's array address (the
 * first call on a device does it too) and keeps it for the process; after a
 * hipDeviceReset that address is stale: call hg_probe_scratch_init again on
 * that device, with it current, before the next hg_root_tactical_probe_noalloc. */
#define HG_PROBE_NOALLOC_MAX_ROOTS 4096
int hg_probe_scratch_init(void);
int hg_root_tactical_probe_noalloc(const uint8_t* states, const uint8_t* legal_moves, const int32_t* num_legal,
                                   const float* priors, int64_t B, int enable_win_in_one,
                                   int enable_check_opponent_wins, int enable_win_in_two, int64_t* winning,
                                   uint8_t* allowed, uint8_t* forced, void* stream);

/* generate_legal_mask_batch / generate_legal_moves_and_mask_batch --
 * game_logic.cu:737-806 (legal_mask_kernel, state_encoder.cuh:908-976).
 * masks[B][85834] f32 (written whole): 1.0 at the action index of every
 * legal slot whose cells fall in the 17x17 window around the centroid, and at
 * PASS_ACTION_INDEX for a PASS.  moves[B][256][6], num_legal[B] as
 * hg_generate_legal_moves; actions[B][256] int32 is scratch (the slots'
 * action indices). */
int hg_legal_mask(const uint8_t* states, int64_t B, uint8_t* moves, int32_t* num_legal, int32_t* actions,
                  float* masks, void* stream);

/* Successor rows of a batch of leaves with the row count kept on the device
 * (no counterpart in the reference, which sizes them on the host:
 * fnn_mcts_orchestrator.py:243-316): offsets[T] int64 = exclusive prefix of
 * the clamped num_legal, total int64 = their sum, the row map (leaf, slot) and
 * features[total][122] of every successor in (leaf, slot) order
 * (fnn_successor_features_kernel semantics, game_logic.cu:182-229).  features
 * must hold T * 256 rows; workspace hg_successor_rows_workspace(T) bytes,
 * 8-byte aligned: offsets, total, then the map. */
int64_t hg_successor_rows_workspace(int64_t T);
int hg_successor_rows(const uint8_t* states, const uint8_t* legal_moves, const int32_t* num_legal, int64_t T,
                      void* workspace, float* features, void* stream);

/* hg_fnn_leaf_eval over the leaves' own legal lists, with no host
 * synchronisation: hg_successor_rows into the workspace, then the network
 * (F = 122; the root rows are root_features [T][122]).  Outputs as
 * hg_fnn_leaf_eval.  workspace: hg_fnn_leaf_eval_lists_workspace(T, F) bytes,
 * 256-byte aligned (the successor rows at capacity T * 256). */
int64_t hg_fnn_leaf_eval_lists_workspace(int64_t T, int F);
int hg_fnn_leaf_eval_lists(const uint8_t* leaf_states, const uint8_t* legal_moves, const int32_t* num_legal,
                           const float* root_features, int64_t T, int F, const float* fc1_w, const float* fc1_b,
                           const float* ln_w, const float* ln_b, const float* fc2_w, const float* fc2_b,
                           const float* value_w, float value_b, const float* action1_w, const float* action1_b,
                           const float* action2_w, float action2_b, void* workspace, float* priors,
                           float* root_values, float* child_q, void* stream);

/* queen_escape_flags_batch -- game_logic.cu:1538-1554.  flags[B] uint8. */
int hg_queen_escape_flags(const uint8_t* states, int64_t B, uint8_t* flags, void* stream);

/* The Gumbel root candidates with their reserve slots, in one launch
 * (FNNMCTSOrchestrator._root_candidate_slots with reserve > 0,
 * hive_fnn/fnn_mcts_orchestrator.py:338-444, there a chain of torch ops over
 * a copy of every child state).  Legal slot j of root r qualifies when its
 * move raises the surround count of the opponent's queen (occupied on-grid
 * neighbours of its cell, 0 while it is unplaced) and, when immobile_only !=
 * 0, the child's side to move has no queen escape (queen_escape_flags_batch
 * on the child).  qualifies (optional): [B][256] uint8, 1 / 0, all 256 slots
 * written.  candidates (optional, then priors [B][256] f32 required):
 * [B][k] int32, columns 0 .. reserve-1 the qualifying slots by prior (-1
 * past their count, at most `reserve`), columns reserve .. k-1 the slots
 * that are legal, allowed (allowed [B][256] uint8, or NULL: all) and not
 * reserved, by prior, followed by the others (ranked at -1e30); every ranking
 * stable (ties to the lower slot).  num_legal is clamped to [0, 256];
 * 1 <= k <= 256, 0 <= reserve <= k. */
int hg_reserve_candidates(const uint8_t* states, const uint8_t* legal_moves, const int32_t* num_legal,
                          const uint8_t* allowed, const float* priors, int64_t B, int k, int reserve,
                          int immobile_only, uint8_t* qualifies, int32_t* candidates, void* stream);

/* The candidate rows of hg_reserve_candidates from given masks: qualifies and
 * valid [B][256] uint8 (nonzero = set), priors [B][256] f32 -> candidates
 * [B][k] int32 (FNNMCTSOrchestrator._root_candidate_slots from its qualifying
 * mask, fnn_mcts_orchestrator.py:411-444). */
int hg_candidate_rows(const uint8_t* qualifies, const uint8_t* valid, const float* priors, int64_t B, int k,
                      int reserve, int32_t* candidates, void* stream);

/* One ply of seeded random play (the position generator of the benchmark
 * configurations; no reference counterpart -- the reference's own pattern is
 * torch.rand x n_legal + apply_moves_batch, hive_gpu/endgame_generator.py:268-276).
 * Game i is active while ply < target_i and its result is 0, where target_i =
 * Philox4x32-10(key=(seed,0), ctr=(i,0,0,0))[0] mod (max_ply+1), or max_ply
 * when lockstep != 0.  An active game applies
 * moves[i][(Philox(key, (i,ply+1,0,0))[0] * num_legal[i]) >> 32] and, when
 * plies_done is not NULL, increments plies_done[i]. */
int hg_random_play_step(uint8_t* states, const uint8_t* moves, const int32_t* num_legal, int64_t B, int ply,
                        int max_ply, int lockstep, uint32_t seed, int32_t* plies_done, void* stream);

/* The plies 0 .. max_ply - 1 of hg_random_play_step (each after the legal
 * lists of hg_generate_legal_moves) in one launch, every game's board held in
 * LDS from its first ply to its last (the state rows receive each ply's
 * changed bytes): the same states and plies_done.  moves: scratch of
 * B * 256 * 6 bytes, required (its first aligned 4-byte word holds the
 * launch's counter of game pairs handed out; calls that share a scratch
 * buffer on different streams race); its contents afterwards are
 * unspecified.  No
 * reference counterpart (the generator of the benchmark configurations, as
 * hg_random_play_step). */
int hg_random_play(uint8_t* states, uint8_t* moves, int64_t B, int max_ply, int lockstep, uint32_t seed,
                   int32_t* plies_done, void* stream);

/* ---------------------------------------------------------------- MCTS tree
 * The reference's structure-of-arrays tree (mcts_tree.cuh:31-45), one pool of
 * max_nodes slots per game, arrays [B, max_nodes] (move_bytes [B, max_nodes, 6],
 * node_count [B]); child_init_q is the extra [B, max_nodes] array the
 * reference passes beside the struct.  Passed by host pointer.
 *
 * Order of effect: simulations of one game take effect in simulation-index
 * order (sim = k*B + game): each selection sees earlier selections' virtual
 * losses, the earliest simulation reaching an unexpanded leaf expands it,
 * node ids are handed out in that order, float updates happen in that order.
 * The reference applies the same updates with atomics in whatever order its
 * threads run. */
typedef struct hg_tree {
    int32_t* visit_count;
    float* total_value;
    float* prior;
    int32_t* parent_idx;
    float* virtual_q_penalty;
    uint8_t* move_bytes;
    int32_t* action_idx;
    int32_t* first_child;
    int32_t* num_children;
    int8_t* is_terminal;
    float* terminal_value;
    int32_t* node_count;
    float* child_init_q;
    int64_t max_nodes;
} hg_tree;

/* ---- legacy action-space engine (hive_gpu/gpu_native_mcts.py; the twelve
 * tree arrays only, no child_init_q).  Same canonical order as below. */

/* mcts_select_batch -- game_logic.cu:961-993 (mcts_select_kernel,
 * mcts_tree.cuh:205-296): PUCT from the root at every level, first maximum,
 * the first child when no score beats -1e30; virtual loss on every entered
 * node.  T = W * B, outputs as hg_mcts_select_root_slots. */
int hg_mcts_select(const hg_tree* tree, const int8_t* game_active, const int32_t* root_nodes, float c_puct, int64_t B,
                   int W, int32_t* leaf_idx, uint8_t* move_paths, int32_t* path_lens, int32_t* vl_paths,
                   int32_t* vl_lens, void* stream);

/* mcts_expand_batch -- game_logic.cu:1018-1045 (mcts_expand_kernel,
 * mcts_tree.cuh:330-433): children for the legal moves that have an action
 * index, prior = action_probs[sim][action] ([T][85834] f32); was_expanded[T]. */
int hg_mcts_expand(const hg_tree* tree, const int32_t* leaf_idx, const uint8_t* leaf_states, const uint8_t* legal_moves,
                   const int32_t* num_legal, const float* action_probs, const int32_t* results, int64_t B,
                   int64_t total, int8_t* was_expanded, void* stream);

/* mcts_backprop_batch -- game_logic.cu:1328-1349 (mcts_backprop_kernel,
 * mcts_tree.cuh:555-605). */
int hg_mcts_backprop(const hg_tree* tree, const int32_t* leaf_idx, const float* nn_values, const int32_t* vl_paths,
                     const int32_t* vl_lens, const int8_t* was_expanded, int64_t B, int64_t total, void* stream);

/* mcts_expand_and_backprop_batch -- game_logic.cu:1053-1080
 * (mcts_expand_and_backprop_kernel, mcts_tree.cuh:435-553). */
int hg_mcts_expand_backprop(const hg_tree* tree, const int32_t* leaf_idx, const uint8_t* leaf_states,
                            const uint8_t* legal_moves, const int32_t* num_legal, const float* action_probs,
                            const int32_t* results, const float* nn_values, const int32_t* vl_paths,
                            const int32_t* vl_lens, int64_t B, int64_t total, void* stream);

/* mcts_extract_policy_batch -- game_logic.cu:1355-1379
 * (mcts_extract_policy_kernel, mcts_tree.cuh:607-687): policies[B][85834]
 * f32, written whole: root visit counts (pruned below pruning_threshold x
 * the maximum, raised to 1/temperature, normalised; uniform when none),
 * one-hot on the most visited child once move_numbers[g] >= temp_drop_move. */
int hg_mcts_extract_policy(const hg_tree* tree, const int32_t* move_numbers, const int32_t* root_nodes,
                           float temperature, int temp_drop_move, float pruning_threshold, int64_t B, float* policies,
                           void* stream);

/* Hard tree rebase of FNNMCTSOrchestrator._reroot_tree
 * (hive_fnn/fnn_mcts_orchestrator.py:1122-1142, rebase_tree_each_move): for
 * each game g with reset[g] != 0, every node of the game's rows returns to
 * its initial fill (visit/value/prior/children/terminal/child_init_q 0,
 * parent/action/first_child -1, move bytes 0; virtual_q_penalty untouched,
 * as in the reference), node_count[g] = 1, root_node[g] = 0.  Only the used
 * prefix [0, node_count[g]) is written: the nodes beyond it still hold the
 * initial fill.  B <= 65535. */
int hg_mcts_reset_trees(const hg_tree* tree, const int8_t* reset, int32_t* root_node, int64_t B, void* stream);

/* mcts_select_with_root_slots_batch -- game_logic.cu:1134-1175
 * (mcts_select_with_root_slots_kernel, mcts_tree.cuh:811-955).
 * T = W * num_candidates * B simulations, sim = (w*C + c)*B + game.
 * Outputs, whole rows written (entries past path_lens / vl_lens are zero, as the
 * reference's zero-filled outputs): leaf_idx[T], move_paths[T][128][6],
 * path_lens[T], vl_paths[T][128], vl_lens[T]. */
int hg_mcts_select_root_slots(const hg_tree* tree, const int8_t* game_active, const int32_t* root_nodes,
                              const int32_t* root_slots, int num_candidates, int max_root_children, float c_puct,
                              int64_t B, int W, int deterministic_non_root, float non_root_sigma, float q_penalty,
                              int32_t* leaf_idx, uint8_t* move_paths, int32_t* path_lens, int32_t* vl_paths,
                              int32_t* vl_lens, void* stream);

/* mcts_select_with_root_mask_batch -- game_logic.cu:1088-1129
 * (mcts_select_with_root_mask_kernel, mcts_tree.cuh:689-800).  T = W * B. */
int hg_mcts_select_root_mask(const hg_tree* tree, const int8_t* game_active, const int32_t* root_nodes,
                             const int8_t* alive_mask, int max_root_children, float c_puct, int64_t B, int W,
                             int deterministic_non_root, float non_root_sigma, float q_penalty, int32_t* leaf_idx,
                             uint8_t* move_paths, int32_t* path_lens, int32_t* vl_paths, int32_t* vl_lens,
                             void* stream);

/* mcts_replay_batch -- game_logic.cu:1000-1015 (mcts_replay_kernel, mcts_tree.cuh:298-320).
 * leaf_states[s] = root_states[s % B] with the path moves applied; rows with
 * leaf_idx < 0 are left untouched. */
int hg_mcts_replay(const uint8_t* root_states, int64_t B, uint8_t* leaf_states, const uint8_t* move_paths,
                   const int32_t* path_lens, const int32_t* leaf_idx, int64_t total, void* stream);

/* The replay step of mcts_select_replay_legal_fnn_root_slots_batch
 * (game_logic.cu:1183-1254), which replays into a zero-filled buffer: as
 * hg_mcts_replay, and rows with leaf_idx < 0 are written as zero rows, so
 * leaf_states may start uninitialised. */
int hg_mcts_replay_fill(const uint8_t* root_states, int64_t B, uint8_t* leaf_states, const uint8_t* move_paths,
                        const int32_t* path_lens, const int32_t* leaf_idx, int64_t total, void* stream);

/* mcts_expand_dense_priors_batch -- game_logic.cu:1259-1288
 * (mcts_expand_dense_priors_kernel, mcts_tree.cuh:971-1062).  was_expanded[total] int8. */
int hg_mcts_expand_dense(const hg_tree* tree, const float* child_q_values, const int32_t* leaf_idx,
                         const uint8_t* leaf_states, const uint8_t* legal_moves, const int32_t* num_legal,
                         const float* priors_per_legal, const int32_t* results, int64_t B, int64_t total,
                         int8_t* was_expanded, void* stream);

/* mcts_expand_and_backprop_dense_priors_batch -- game_logic.cu:1293-1323
 * (mcts_expand_and_backprop_dense_priors_kernel, mcts_tree.cuh:1068-1187). */
int hg_mcts_expand_backprop_dense(const hg_tree* tree, const float* child_q_values, const int32_t* leaf_idx,
                                  const uint8_t* leaf_states, const uint8_t* legal_moves, const int32_t* num_legal,
                                  const float* priors_per_legal, const int32_t* results, const float* nn_values,
                                  const int32_t* vl_paths, const int32_t* vl_lens, float q_penalty, int64_t B,
                                  int64_t total, void* stream);

/* hg_mcts_expand_backprop_dense with a workspace of
 * hg_mcts_expand_backprop_dense_workspace(B, total) bytes (4-byte aligned;
 * accepted and not written: the plan lives in on-chip memory): the same
 * tree, the simulations of different root children applied in parallel (one
 * workgroup per game: a planning wave settles node ids and the root's
 * statistics in simulation order, then one wave per root child).  Identical
 * results; the
 * one-wave-per-game order is kept for games whose node pool could run short
 * or with a path that is not a selection path (each entry a node of the pool
 * whose parent is the entry before it, the last entry the leaf).  Path
 * entries are node ids below max_nodes, as in the reference. */
int64_t hg_mcts_expand_backprop_dense_workspace(int64_t B, int64_t total);
int hg_mcts_expand_backprop_dense_ws(const hg_tree* tree, const float* child_q_values, const int32_t* leaf_idx,
                                     const uint8_t* leaf_states, const uint8_t* legal_moves,
                                     const int32_t* num_legal, const float* priors_per_legal, const int32_t* results,
                                     const float* nn_values, const int32_t* vl_paths, const int32_t* vl_lens,
                                     float q_penalty, int64_t B, int64_t total, void* workspace, void* stream);

/* mcts_apply_root_noise -- game_logic.cu:1384-1402 (mcts_root_noise_kernel,
 * mcts_tree.cuh:1192-1234).  noise[B][max_children_pad]; children beyond the
 * pad are left unchanged (the reference reads past the row there). */
int hg_mcts_root_noise(const hg_tree* tree, const float* noise, const int32_t* root_nodes, int max_children_pad,
                       float dir_eps, float root_policy_temp, int64_t B, void* stream);

/* Search counters of one simulation wave (no counterpart in the reference:
 * instrumentation for throughput accounting).  Over rows t < total with
 * leaf_idx[t] >= 0: stats[0] += 1, stats[1] += num_legal[t], stats[2] +=
 * vl_lens[t]; and stats[3] += total.  stats is int64[4] in device memory,
 * updated in stream order (calls on one stream accumulate). */
int hg_mcts_wave_stats(const int32_t* leaf_idx, const int32_t* num_legal, const int32_t* vl_lens, int64_t total,
                       int64_t* stats, void* stream);

/* One decision of the Gumbel root search's sequential halving
 * (fnn_mcts_orchestrator.py:650-731: the statistics of the candidates' root
 * children, the batch-global sigma, the scores and the survivors; no single
 * reference entry point -- the reference runs these as torch ops between
 * rounds).  candidates[B][C] root slots (-1 = none), 1 <= C <= 64; base[B][256]
 * the Gumbel draw + legal logit of every slot.  A column's visits N and Q
 * (-W / max(N, 1) when N > root_q_min_visits, else 0) are those of the root
 * child in its slot (0, 0 outside the root's children); sigma = (c_visit + the
 * largest candidate N of the batch) * c_scale; score = base[g][slot] + sigma *
 * Q, -1e30 for an empty column.  keep > 0 (= C / 2 between rounds): the
 * columns in descending score order (ties to the lower column), the first
 * keep written to cand_out[B][keep] -- the first max(1, nonempty / 2) as
 * their slots, the rest -1.  keep = 0 (the final choice): chosen[g] = the
 * slot of the first highest column, 0 when it is empty. */
int hg_gumbel_halving(const hg_tree* tree, const int32_t* root_nodes, const int32_t* candidates, int C,
                      const float* base, float c_visit, float c_scale, int root_q_min_visits, int keep, int64_t B,
                      int32_t* cand_out, int64_t* chosen, void* stream);

/* ---- one simulation wave of the Gumbel root search, launched natively ----
 * The body of the reference's per-wave loop (fnn_mcts_orchestrator.py:982-1055:
 * mcts_select_replay_legal_fnn_root_slots_batch, the FNN leaf evaluation,
 * mcts_expand_and_backprop_dense_priors_batch) as one host call: select over
 * the root slots -> replay (rows of idle simulations zero) and the leaves'
 * results -> legal lists + features -> hg_fnn_leaf_eval_lists -> expansion +
 * backup (hg_mcts_expand_backprop_dense_ws), launched in that order on
 * `stream` with no host synchronisation and no allocation.  No single
 * reference entry point: it saves the host the per-call argument handling of
 * six entry points per wave.  Results are those of the six calls. */
typedef struct hg_fnn_net {   /* a 64-wide HiveFNN (fnn_network.py:97-140), F = 122 */
    const float* fc1_w;       /* [64][F] */
    const float* fc1_b;       /* [64] */
    const float* ln_w;        /* [64] */
    const float* ln_b;        /* [64] */
    const float* fc2_w;       /* [64][64] */
    const float* fc2_b;       /* [64] */
    const float* value_w;     /* [64] */
    const float* action1_w;   /* [64][128] */
    const float* action1_b;   /* [64] */
    const float* action2_w;   /* [64] */
    float value_b;
    float action2_b;
    int32_t F;
} hg_fnn_net;

typedef struct hg_wave_buffers {  /* rows for T = W * num_candidates * B simulations (or more) */
    int32_t* leaf_idx;       /* [T] */
    uint8_t* move_paths;     /* [T][128][6], each row written up to its path_lens entry */
    int32_t* path_lens;      /* [T] */
    int32_t* vl_paths;       /* [T][128], each row written up to its vl_lens entry */
    int32_t* vl_lens;        /* [T] */
    uint8_t* leaf_states;    /* [T][3424] */
    int32_t* results;        /* [T] */
    uint8_t* legal_moves;    /* [T][256][6], each row written up to its num_legal entry */
    int32_t* num_legal;      /* [T] */
    float* features;         /* [T][122], 8-byte aligned */
    float* priors;           /* [T][256], each row written up to its leaf's legal count */
    float* values;           /* [T] */
    float* child_q;          /* [T][256], each row written up to its leaf's legal count */
    void* leaf_workspace;    /* hg_fnn_leaf_eval_lists_workspace(T, 122) bytes, 256-byte aligned */
    void* tree_workspace;    /* hg_mcts_expand_backprop_dense_workspace(B, T) bytes, 4-byte aligned */
    int64_t* stats;          /* NULL, or hg_mcts_wave_stats' int64[4], accumulated */
    int64_t capacity;        /* rows each [T] array above holds */
} hg_wave_buffers;

int hg_mcts_wave_root_slots(const hg_tree* tree, const uint8_t* root_states, const int8_t* game_active,
                            const int32_t* root_nodes, const int32_t* root_slots, int num_candidates,
                            int max_root_children, float c_puct, int64_t B, int W, int deterministic_non_root,
                            float non_root_sigma, float q_penalty, const hg_fnn_net* net,
                            const hg_wave_buffers* buffers, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HIVE_GPU_H */
