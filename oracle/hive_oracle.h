/*
 * hive_oracle.h -- C-ABI of the CPU oracle.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * product path: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  Nothing in hive_neuralnet_amd/ links or calls it.
 *
 * Byte formats are the reference's wire formats:
 *   state : 3424 bytes, HiveState layout (hive_gpu/csrc/hive_state.cuh:239-269)
 *   move  : 6 bytes {u8 type, u8 piece_type, u16 from, u16 to} little-endian
 *           (hive_gpu/csrc/hive_state.cuh:228-233)
 */
#ifndef HIVE_ORACLE_H
#define HIVE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_STATE_BYTES 3424
#define OR_MOVE_BYTES 6
#define OR_MAX_LEGAL 256
#define OR_FEAT_DIM 122

int or_state_bytes(void);

/* single-state primitives */
void or_init_state(uint8_t* state, int expansion_mask);
void or_apply_move(uint8_t* state, const uint8_t* move6);
int or_legal_moves(const uint8_t* state, uint8_t* moves_out /* 256*6, fully written */);
int or_fnn_feature_moves(const uint8_t* state, uint8_t* moves_out /* 256*6 */);
void or_fnn_features(const uint8_t* state, const uint8_t* moves, int n, float* feat_out);
void or_articulation(const uint8_t* state, uint64_t* ap_out /* 9 words */);
void or_centroid(const uint8_t* state, int* cq, int* cr);
int or_move_to_action(const uint8_t* move6, int cq, int cr);
int or_queen_escape(const uint8_t* state);
void or_neighbor_table(int16_t* out /* 529*6 */);

/* batched helpers (threads <= 0 means 1) */
void or_batch_legal_features_actions(const uint8_t* states, int64_t B,
                                     uint8_t* moves_out, int32_t* n_out,
                                     float* feat_out, int32_t* act_out,
                                     int threads);
void or_batch_successor_features(const uint8_t* states, const uint8_t* legal,
                                 const int64_t* action_to_root,
                                 const int64_t* move_indices, int64_t N,
                                 float* feat_out, int full_list, int threads);
void or_batch_queen_escape(const uint8_t* states, int64_t B, uint8_t* out, int threads);
/* root_tactical_probe_batch (game_logic.cu:290-397): nlegal clamped by the caller to <= 256 */
void or_batch_root_tactical_probe(const uint8_t* states, const uint8_t* legal, const int32_t* nlegal,
                                  const float* priors, int64_t B, int win1, int screen, int win2, int64_t* win,
                                  uint8_t* allowed, uint8_t* forced, int threads);
int or_surround_count(const uint8_t* state, int colour);
int or_immediate_win(const uint8_t* state);

/* Philox4x32-10 and the seeded random-play position generator */
void or_philox4x32_10(uint32_t key0, uint32_t key1, const uint32_t ctr[4], uint32_t out[4]);
void or_generate_positions(int64_t B, int expansion_mask, int max_ply, uint32_t seed,
                           uint8_t* states_out, int32_t* plies_out, int threads);
void or_lockstep_selfplay(int64_t G, int expansion_mask, int max_ply, uint32_t seed,
                          uint8_t* states_out, int32_t* plies_out, int threads);

/* MCTS tree (hive_mcts_oracle.c): host arrays in the reference's SoA layout */
typedef struct {
    int32_t* vc;   /* visit_count [B, M] */
    float* tv;     /* total_value */
    float* pr;     /* prior */
    int32_t* pa;   /* parent_idx */
    float* vq;     /* virtual_q_penalty */
    uint8_t* mb;   /* move_bytes [B, M, 6] */
    int32_t* ai;   /* action_idx */
    int32_t* fc;   /* first_child */
    int32_t* nc;   /* num_children */
    int8_t* it;    /* is_terminal */
    float* tval;   /* terminal_value */
    int32_t* cnt;  /* node_count [B] */
    float* ciq;    /* child_init_q */
    int64_t M;     /* max_nodes */
} or_tree;

void or_mcts_select_slots(const or_tree* t, const int8_t* active, const int32_t* roots, const int32_t* slots, int C,
                          int max_root, float c_puct, int64_t B, int W, int det, float sigma, float qp,
                          int32_t* leaf, uint8_t* paths, int32_t* plen, int32_t* vl, int32_t* vlen);
void or_mcts_select_mask(const or_tree* t, const int8_t* active, const int32_t* roots, const int8_t* alive,
                         int max_root, float c_puct, int64_t B, int W, int det, float sigma, float qp,
                         int32_t* leaf, uint8_t* paths, int32_t* plen, int32_t* vl, int32_t* vlen);
void or_mcts_replay(const uint8_t* roots, int64_t B, uint8_t* leaves, const uint8_t* paths, const int32_t* plen,
                    const int32_t* leaf, int64_t total);
void or_mcts_expand_dense(const or_tree* t, const float* child_q, const int32_t* leaf, const uint8_t* states,
                          const uint8_t* legal, const int32_t* nlegal, const float* priors, const int32_t* results,
                          int64_t B, int64_t total, int8_t* was);
void or_mcts_expand_backprop_dense(const or_tree* t, const float* child_q, const int32_t* leaf, const uint8_t* states,
                                   const uint8_t* legal, const int32_t* nlegal, const float* priors,
                                   const int32_t* results, const float* values, const int32_t* vl,
                                   const int32_t* vlen, float qp, int64_t B, int64_t total);
void or_mcts_root_noise(const or_tree* t, const float* noise, const int32_t* roots, int pad, float eps, float temp,
                        int64_t B);
/* legacy action-space engine (mcts_tree.cuh:205-687) */
void or_mcts_select_legacy(const or_tree* t, const int8_t* active, const int32_t* roots, float c_puct, int64_t B,
                           int W, int32_t* leaf, uint8_t* paths, int32_t* plen, int32_t* vl, int32_t* vlen);
void or_mcts_expand_legacy(const or_tree* t, const int32_t* leaf, const uint8_t* states, const uint8_t* legal,
                           const int32_t* nlegal, const float* probs, const int32_t* results, int64_t B, int64_t total,
                           int8_t* was);
void or_mcts_backprop_legacy(const or_tree* t, const int32_t* leaf, const float* values, const int32_t* vl,
                             const int32_t* vlen, const int8_t* was, int64_t B, int64_t total);
void or_mcts_expand_backprop_legacy(const or_tree* t, const int32_t* leaf, const uint8_t* states,
                                    const uint8_t* legal, const int32_t* nlegal, const float* probs,
                                    const int32_t* results, const float* values, const int32_t* vl,
                                    const int32_t* vlen, int64_t B, int64_t total);
void or_mcts_extract_policy(const or_tree* t, const int32_t* move_numbers, const int32_t* roots, float temperature,
                            int temp_drop, float pruning, int64_t B, float* policies);
void or_legal_mask(const uint8_t* states, const uint8_t* legal, const int32_t* nlegal, int64_t B, float* masks);

/* CPU search player (hive_cpu_player.c): FNNNativeCPUPlayer's serial Gumbel
 * search (hive_fnn/fnn_native_cpu_player.py:126-266), one game per thread.
 * Weights of the `large` network in torch's layout (Linear weight [out, in]). */
typedef struct {
    const float *fc1_w, *fc1_b, *ln_w, *ln_b, *fc2_w, *fc2_b, *value_w;
    float value_b;
    const float *a1_w, *a1_b, *a2_w;
    float a2_b;
} or_fnn_weights;
void or_cpu_player_search(const uint8_t* states, int64_t G, const or_fnn_weights* w, int num_sims, int considered,
                          float c_puct, float c_visit, float c_scale, int32_t* chosen, int64_t* sims, int threads);

#ifdef __cplusplus
}
#endif

#endif
