/*
 * jq_oracle.h -- CPU restatement of the junqi_core rules (test infrastructure).
 *
 * THIS IS THE ORACLE. It exists only to check the HIP implementation in
 * junqi_amd/: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * are the only callers. Nothing in the product links or loads it.
 *
 * Every function restates the behaviour of one reference function and cites it
 * (paths relative to the reference repository). Semantic authority is
 * junqi_core/state.py::GameState; where BatchedGameState diverges from it,
 * GameState's behaviour is the one restated.
 *
 * How it is pinned (tests/test_oracle*.py): the reference's golden scenarios,
 * observation hashes and recorded game; its known-answer tests (rotation,
 * combat memory, beliefs, setup validation) restated; the 4-fold rotation
 * symmetry of the rules; and 12 complete reference games (Zobrist hash after
 * every ply; combat memory, beliefs and all four observers' float32
 * observations bit for bit at seven plies each, BRIGHT / DARK / HALF_DARK)
 * written by tests/golden/gen_reference_vectors.py.
 */
#ifndef JQ_ORACLE_H
#define JQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JQO_NC 289   /* 17x17 flat cells */
#define JQO_NP 120   /* piece ids: seat*30 + slot */
#define JQO_OBS_C 317
#define JQO_OBS_G 28
#define JQO_ONB 129  /* on-board cells */
#define JQO_SLOTS 80 /* per-piece legal slots (game_state.cu:1969) */

/* PieceType values (junqi_core/rules.py:49-70) */
enum { JQO_NONE = 0, JQO_DARK = 1, JQO_JUNQI = 2, JQO_DILEI = 3, JQO_ZHADAN = 4,
       JQO_SILING = 5, JQO_JUNZH = 6, JQO_SHIZH = 7, JQO_LVZH = 8, JQO_TUANZH = 9,
       JQO_YINGZH = 10, JQO_LIANZH = 11, JQO_PAIZH = 12, JQO_GONGB = 13 };
/* Event (rules.py:283-289); 0 = invalid / no step */
enum { JQO_EV_NONE = 0, JQO_EV_MOVE = 1, JQO_EV_EAT = 2, JQO_EV_BOMB = 3, JQO_EV_KILLED = 4 };
/* ShowMode (rules.py:453-458) */
enum { JQO_BRIGHT = 0, JQO_DARKMODE = 1, JQO_HALF_DARK = 2 };

typedef struct jqo_game {
    /* piece-indexed SoA (state.py:301-316) */
    int8_t  alive[JQO_NP], ptype[JQO_NP], pseat[JQO_NP];
    int8_t  pos_x[JQO_NP], pos_y[JQO_NP], zero_x[JQO_NP], zero_y[JQO_NP];
    int16_t move_count[JQO_NP], active_eat[JQO_NP], passive_surv[JQO_NP];
    int8_t  death_reason[JQO_NP];
    int16_t death_step[JQO_NP], death_loc[JQO_NP];
    int16_t cell_pid[JQO_NC];
    int8_t  seat_dead[4], flag_rev[4];
    int8_t  turn, terminated, winner, draw, show_mode, pad_[3];
    int32_t move_counter, mslc, max_num_moves;
    uint64_t zobrist;
    /* move history, most recent last, at most 32 entries (state.py:673-678) */
    int16_t hist[32][2];
    int32_t hist_len;
    /* CombatMemory v6, [observer][pid] (combat_memory.py:251-311) */
    uint64_t cm_direct_lo[4][JQO_NP], cm_direct_hi[4][JQO_NP];
    uint16_t cm_direct_type[4][JQO_NP];
    int16_t  cm_last_direct[4][JQO_NP], cm_other_cnt[4][JQO_NP];
    uint64_t cm_chain_lo[4][JQO_NP], cm_chain_hi[4][JQO_NP];
    uint16_t cm_chain_type[4][JQO_NP];
    int16_t  cm_last_chain[4][JQO_NP];
    uint64_t cm_eaten_lo[4][JQO_NP], cm_eaten_hi[4][JQO_NP];
    int8_t   cm_floor[4][JQO_NP];
    int16_t  cm_floor_step[4][JQO_NP];
    int8_t   cm_is_gongb[4][JQO_NP], cm_not_gongb[4][JQO_NP], cm_atk_gongb[4][JQO_NP];
    /* BeliefTensor per observer, held as row codes (info_model.py:164-561):
     * 0 zero row, 1..12 one-hot(tracked type idx + 1), 16+slot prior row,
     * 64 uniform. rem_tracked[o][s] says whether remaining[s] exists. */
    uint8_t bcode[4][JQO_NP];
    int8_t  rem_tracked[4][4];
    int16_t rem[4][4][12];
} jqo_game;

typedef struct jqo_result {
    int32_t valid, event, flag_reveal_src, flag_reveal_dst, flag_captured;
    int32_t seats_died_mask, terminated, winner, draw, gongb_revealed;
} jqo_result;

/* ---- tables / topology ---- */
void jqo_init(void);
void jqo_tables_export(int8_t *on_board, int8_t *is_rail, int8_t *is_camp,
                       int8_t *is_stronghold, int8_t *is_ninegrid, int8_t *curve_id,
                       int8_t *curve_arc, int16_t *compact_to_flat, int16_t *rail_adj4);

/* ---- CPython random.Random restatement (stdlib, not vendored) ---- */
typedef struct jqo_mt { uint32_t mt[624]; int idx; } jqo_mt;
void     jqo_mt_seed(jqo_mt *r, uint64_t seed);
uint32_t jqo_mt_u32(jqo_mt *r);
uint32_t jqo_mt_randbelow(jqo_mt *r, uint32_t n);
void     jqo_random_lineup(jqo_mt *r, int8_t lineup[30]);
void     jqo_random_setup(uint64_t seed, int8_t setup[120]);
void     jqo_setup_pool(uint64_t seed, int32_t pool_size, int8_t *pool /* pool_size*120 */);

/* ---- numpy PCG64 restatement (Zobrist tables, junqi_core/_zobrist.py:73-122) ---- */
void     jqo_seedseq_state(uint64_t entropy, uint32_t out8[8]);
void     jqo_pcg64_draw(uint64_t seed, int64_t n, uint64_t *out);
int64_t  jqo_zobrist_count(void);
const uint64_t *jqo_zobrist_all(void);

/* ---- recency LUT (float32 exp(-e/tau) as numpy computes it; fixture data) ---- */
void jqo_set_recency_lut(const float *lut4x4096);

/* ---- game ---- */
int  jqo_new_game(jqo_game *g, const int8_t setup[120], int show_mode, int max_num_moves);
int  jqo_from_pieces(jqo_game *g, int n, const int32_t *pieces /* n x (pid, type, x, y) */,
                     int turn, int move_counter, int mslc, const int8_t seat_dead[4],
                     const int8_t flag_rev[4], int show_mode, int max_num_moves);
int  jqo_is_legal(const jqo_game *g, int seat, int src, int dst);
int  jqo_legal_ids(const jqo_game *g, int seat, int32_t *out, int cap);
int  jqo_has_legal(const jqo_game *g, int seat);
/* Per-piece 80-slot legal mask of `seat` (game_state.cu:1964-2197), out[120*80]:
 * slots 0-3 road steps (+x,-x,+y,-y), 4-7 camp diagonals, 8-55 straight rail
 * runs (dir*12 + k), 56-67 curve-rail destinations in BFS order, engineers'
 * rail BFS destinations from slot 8. Zero for a dead seat or a finished game,
 * like jqo_legal_ids. Returns the number of set slots. */
int  jqo_legal_slots(const jqo_game *g, int seat, uint8_t *out);
int  jqo_step(jqo_game *g, int src, int dst, jqo_result *res);
int  jqo_move_requires_gongb(const jqo_game *g, int src, int dst);
void jqo_observe(const jqo_game *g, int observer, float *spatial /*317*289*/, float *glob /*28*/);
/* The same with the belief planes (12-23, 27-50) taken from the observer's
 * uploaded (12, 289) world-cell belief slice: value at each teammate / enemy
 * piece's cell where > 0 (observation.cu:246-372); globals unchanged. */
void jqo_observe_ext(const jqo_game *g, int observer, const float *ext /*12*289*/, float *spatial, float *glob);
uint64_t jqo_recompute_zobrist(const jqo_game *g);
void jqo_belief_row(int code, float out[12]);

/* ---- rotation (rotation.py:44-80), placement (board.py:88-102), action codec ---- */
void jqo_world_to_canonical(int x, int y, int seat, int *cx, int *cy);
void jqo_canonical_to_world(int cx, int cy, int seat, int *x, int *y);
void jqo_index_to_pos(int seat, int i, int *x, int *y);
/* compact canonical id FLAT_TO_COMPACT[rot(src)]*129 + FLAT_TO_COMPACT[rot(dst)] of a world id */
int  jqo_canonical_id(int seat, int world_id);

/* ---- setup validation (setup.py:60-136) ---- */
#define JQO_V_TYPE 1   /* a value that is not a PieceType */
#define JQO_V_C1 2     /* camp not empty */
#define JQO_V_C2 4     /* not exactly one flag, or flag outside a stronghold */
#define JQO_V_C3 8     /* landmine outside the back two rows */
#define JQO_V_C4 16    /* bomb in the front row */
#define JQO_V_C5 32    /* piece counts */
int  jqo_validate_lineup(const int8_t lineup[30]);

/* ---- CombatMemory on hand-built cases (combat_memory.py:339-569) ---- */
void jqo_cm_apply_event(jqo_game *g, int is_eat, int apid, int dpid, int aseat, int dseat, int atype, int dtype,
                        int step);
void jqo_cm_path_revealed_gongb(jqo_game *g, int pid);

/* ---- samplers (Philox4x32-10, Salmon et al. SC'11) ---- */
void    jqo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
int32_t jqo_sample_uniform(const int32_t *ids, int n, int env, uint64_t seed, uint64_t ply);
int32_t jqo_sample_logits(const int32_t *ids, int n, int seat, int env, uint64_t seed, uint64_t ply,
                          int32_t *canon);
int32_t jqo_reset_pool_index(int env, int64_t seed, int pool_size);

/* ---- batch (CPU baseline; OpenMP over envs) ---- */
int  jqo_sizeof_game(void);
int  jqo_omp_threads(void);
void jqo_batch_new(jqo_game *gs, int n, const int8_t *setups, int show_mode, int max_num_moves);
/* One env-step per env: step with actions[i] (world id src*289+dst, -1 = skip),
 * then legal ids for the new turn, canonical bitmask and the acting seat's obs.
 * Returns total legal-id count. */
long jqo_batch_env_step(jqo_game *gs, int n, const int32_t *actions, int32_t *legal_counts,
                        uint8_t *mask_bits, float *obs_spatial, float *obs_global, int write_obs);

/* Rollout: `steps` env-steps of sample (0 uniform, 1 masked logits; games with
 * k < active_from[i] take no action) -> step -> record reward / done / hash ->
 * restart finished games from the pool -> count and digest the new legal row.
 * Outputs (steps, n) row-major, any may be NULL. */
long jqo_batch_rollout(jqo_game *gs, int n, const int8_t *pool, int pool_size, int sampler, uint64_t seed,
                       uint64_t ply0, int64_t reset_seed0, int steps, const int32_t *active_from, float *reward,
                       uint8_t *done, uint64_t *hash, int32_t *actions, int32_t *legal_count,
                       uint64_t *legal_digest);
/* The CPU baseline's env-step: sample from the ids left by the previous call,
 * step, restart from the pool, new legal ids + canonical mask + f32 observation
 * (OpenMP over games; ply < 0 only fills the opening ids). */
long jqo_batch_cpu_env_step(jqo_game *gs, int n, const int8_t *pool, int pool_size, int sampler, uint64_t seed,
                            int64_t ply, int64_t reset_seed, int32_t *ids, int cap, int32_t *counts,
                            uint8_t *mask_bits, float *obs_spatial, float *obs_global);
/* OpenMP thread count of the batch functions (n > 0). */
void jqo_set_threads(int n);
/* Acting-seat observations of games [g0, g1), rows from 0 (OpenMP). */
void jqo_batch_observe(const jqo_game *gs, int g0, int g1, float *spatial, float *glob);

#ifdef __cplusplus
}
#endif
#endif
