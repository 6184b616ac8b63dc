/*
 * junqi_amd.h -- C ABI of the MI355X batched Junqi environment.
 *
 * One handle owns N games in HBM. Every entry point returns 0 on success or a
 * negative JQ_E* code (message via jq_last_error()); nothing throws or exits.
 * Device pointers are plain addresses of caller memory (e.g. torch tensors);
 * `stream` is a hipStream_t passed as void* (NULL = default stream). No entry
 * point synchronises the device unless it says so.
 *
 * Each declaration names the reference interface it replaces (paths relative
 * to the reference repository).
 */
#ifndef JUNQI_AMD_H
#define JUNQI_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JQ_NUM_CELLS 289
#define JQ_NUM_ON_BOARD 129
#define JQ_NUM_PIDS 120
#define JQ_OBS_CHANNELS 317
#define JQ_OBS_GLOBALS 28
#define JQ_ACTION_DIM 16641        /* 129 * 129 compact canonical actions */
#define JQ_MASK_WORDS 521          /* 32-bit words per packed canonical mask row */
#define JQ_AUX_BYTES 2320          /* u8 aux row: float32[2] turn history + uint16[4][289] recency codes */
#define JQ_MAX_LEGAL 3200          /* per-env upper bound on legal actions (25 pieces x 128) */
/* setup styles for jq_generate_styled */
#define JQ_SETUP_CANONICAL 1
#define JQ_SETUP_MIXED 2
#define JQ_SLOTS_PER_PIECE 80      /* per-piece legal slot mask width (game_state.cu:1969) */

/* error codes */
#define JQ_OK 0
#define JQ_E_ARG (-1)      /* bad argument (null, range, shape) */
#define JQ_E_STATE (-2)    /* handle not ready (tables / pool missing) */
#define JQ_E_HIP (-3)      /* HIP runtime error */
#define JQ_E_OOM (-4)      /* device allocation failed */
#define JQ_E_CAPACITY (-5) /* an output buffer is smaller than the result */

/* lineup violation bits of jq_validate_lineup (setup.py:60-136) */
#define JQ_LINEUP_TYPE 1   /* a value that is not a PieceType (0..13) */
#define JQ_LINEUP_C1 2     /* a camp slot holds a piece */
#define JQ_LINEUP_C2 4     /* not exactly one flag, or the flag outside the strongholds */
#define JQ_LINEUP_C3 8     /* a landmine outside the back two rows */
#define JQ_LINEUP_C4 16    /* a bomb in the front row */
#define JQ_LINEUP_C5 32    /* piece counts differ from PIECE_COUNTS */

/* samplers of jq_env_step */
#define JQ_SAMPLE_UNIFORM 0 /* Philox pick uniform over the legal CSR row */
#define JQ_SAMPLE_LOGITS 1  /* argmax of i.i.d. N(0,1) logits over the legal canonical ids */

/* observation output formats */
#define JQ_OBS_F32 0       /* (N,317,17,17) float32, the reference layout */
#define JQ_OBS_BF16 1      /* (N,317,17,17) bfloat16 = round-to-nearest-even of the f32 */
#define JQ_OBS_U8 2        /* (N,317,17,17) uint8 codes + (N,JQ_AUX_BYTES) aux rows, see jq_observe */

/* action formats for jq_step */
#define JQ_ACT_WORLD 0     /* src_flat*289 + dst_flat in the world frame */
#define JQ_ACT_CANONICAL 1 /* compact canonical id src_c*129 + dst_c of the acting seat */

typedef struct jq_env jq_env;

/* Last error message of the calling thread. */
const char *jq_last_error(void);
/* Library version string. */
const char *jq_version(void);

/* Create / destroy N games on `device`. Replaces junqi_cuda.DeviceGameStateBatch
 * (src/env/cuda/src/bindings.cpp:462-560) and DeviceObservation*Batch. */
int jq_create(jq_env **out, int32_t num_envs, int32_t max_num_moves, int32_t show_mode, int32_t device);
int jq_destroy(jq_env *env);
int32_t jq_num_envs(const jq_env *env);

/* Zobrist tables as numpy's PCG64 stream draws them (junqi_core/_zobrist.py:80-106),
 * host pointer, `count` uint64 values. Replaces junqi_cuda.upload_zobrist_tables
 * (junqi_rl/gpu_world.py:77-94). Must precede any reset. */
int jq_upload_zobrist(jq_env *env, const uint64_t *host_table, int64_t count);

/* Recency table float32[4][4096] (observation.py:1552-1567 values). Host pointer. */
int jq_upload_recency(jq_env *env, const float *host_lut);

/* validate_lineup (junqi_core/setup.py:60-136) of one seat's 30 slot types:
 * returns 0 when C1-C5 hold, else the JQ_LINEUP_* bits of every rule broken
 * (JQ_LINEUP_TYPE alone when a value is not a PieceType), or JQ_E_ARG for a
 * null pointer. Host only. */
int jq_validate_lineup(const int8_t *lineup30);

/* Setup pool (pool_size,120) int8 piece types per pid, host pointer. Every
 * seat's lineup must pass jq_validate_lineup, else JQ_E_ARG names the first
 * bad entry and the handle keeps its previous pool. The pool buffer is
 * reused while the new pool fits and replaced (after a device sync) when it
 * grows, so repeated uploads hold one buffer. Replaces
 * junqi_cuda.upload_setup_pool (junqi_rl/gpu_rollout.py:588-652). */
int jq_upload_setup_pool(jq_env *env, const int8_t *host_pool, int32_t pool_size);

/* Start every env from the given lineups ((N,120) int8 piece types per pid, host
 * pointer): GameState.new_game + BeliefTensor.initial for all four observers.
 * Lineups are validated as GameState.new_game does (state.py:498-507): a
 * violation returns JQ_E_ARG naming the env and seat, and no env is touched.
 * Replaces GpuRollout.reset's copy_from_host path (junqi_rl/gpu_rollout.py:690-744).
 * A CSR from before the reset no longer describes the games: call jq_legal
 * before sampling from one (jq_env_step's sampler reads the CSR it is given). */
int jq_reset_lineups(jq_env *env, const int8_t *host_lineups, void *stream);

/* Host-side lineup generation identical to junqi_core.setup.generate_random_setup
 * (setup.py:162-258) under random.Random(seed_base + i), then jq_reset_lineups.
 * This is GpuRollout.reset(seed_base) (gpu_rollout.py:690-744). Synchronises. */
int jq_reset_seeded(jq_env *env, int64_t seed_base, void *stream);
/* The lineups jq_reset_seeded would use, without touching the device. */
int jq_generate_lineups(int64_t seed_base, int32_t count, int8_t *host_out);
/* The setup pool of junqi_rl/gpu_rollout.py:255-275: pool_size setups drawn from
 * one random.Random(seed) stream, (pool_size,120) int8 piece types per pid. */
int jq_generate_pool(int64_t seed, int32_t pool_size, int8_t *host_out);
/* Canonical and mixed setup styles of GpuRollout (gpu_rollout.py:498-560).
 * mode JQ_SETUP_CANONICAL: every seat takes the lineup of a style drawn with
 * random.choice from `styles` (_build_canonical_pool, gpu_rollout.py:278-306);
 * JQ_SETUP_MIXED: seats 0 and 2 take it, seats 1 and 3 draw uniform-random
 * lineups in seat order (_build_mixed_pool, gpu_rollout.py:309-382). styles:
 * nstyles letters of "TDGF" (CANONICAL_LINEUPS, setup_canonical.py:264-269)
 * in the caller's order. per_game_seed != 0: setup i draws from
 * random.Random(seed + i), as GpuRollout.reset (gpu_rollout.py:701-728); else
 * all setups come from one random.Random(seed) stream, as the pool builders.
 * host_out: (count, 120) int8 piece types per pid. Host only. */
int jq_generate_styled(int32_t mode, int64_t seed, int32_t count, int32_t per_game_seed, const char *styles,
                       int32_t nstyles, int8_t *host_out);
/* Copy of the host-built constant board tables (struct jq::Tables of
 * junqi_amd/csrc/jq_topology.h), for inspection by tests. */
int jq_board_tables(void *host_out, int64_t nbytes);

/* Reset terminated envs from the pool, picking entry hash(env, seed) % pool_size
 * (src/env/cuda/src/game_state.cu:2936-3102). Replaces reset_terminated_envs
 * (gpu_rollout.py:1007-1028). */
int jq_reset_terminated(jq_env *env, int64_t seed, void *stream);

/* Apply one ply per env. actions: device int32 (N) in `action_format`; acting:
 * device int8 (N) seat per env (NULL = current turn; required for canonical ids).
 * Outputs (device, any may be NULL): valid u8, event i8, terminated u8, winner i8,
 * draw u8, flag_captured u8, seats_died u8 bitmask, reward f32 (acting team +-1 on
 * the ply that ends the game), world_action i32.
 * Replaces step_device (game_state.cu:2731-2797, bindings.cpp:1044-1073) and
 * GpuWorld.step_batch (gpu_world.py:223-253). Terminated envs are skipped. */
int jq_step(jq_env *env, const int32_t *actions, const int8_t *acting, int32_t action_format,
            uint8_t *valid, int8_t *event, uint8_t *terminated, int8_t *winner, uint8_t *draw,
            uint8_t *flag_captured, uint8_t *seats_died, float *reward, int32_t *world_action,
            void *stream);

/* Legal actions of `acting` (device int8 N; NULL = current turn) for every env.
 * counts: device int32 (N); offsets: device int32 (N+1), exclusive scan of counts;
 * values: device int32 of values_capacity elements, per-env ascending world ids
 * src*289+dst (move_gen.py:1199 order); mask_words: device int32 (N, 521) packed
 * canonical compact mask; mask_bool: device uint8 (N, 16641) (gpu_rollout.py:1220).
 * Any output may be NULL (offsets/values need counts). values_capacity >=
 * N*JQ_MAX_LEGAL can never overflow, and for N <= 671,088 (where that bound fits
 * the int32 offsets) the call stays asynchronous; otherwise the call reads the
 * total (offsets[N]) back, as the reference's CSR call does
 * (game_state.cu:1936-1948), and returns JQ_E_CAPACITY without writing values
 * when the ids do not fit the buffer or their total exceeds INT32_MAX (offsets
 * and counts are written; offsets[N] is then -1). No kernel writes outside
 * values[0 .. values_capacity). Replaces legal_action_ids_batch_csr
 * (game_state.cu:1892-1962) and legal_mask_canonical_batch (game_state.cu:2291-2508). */
int jq_legal(jq_env *env, const int8_t *acting, int32_t *counts, int32_t *offsets, int32_t *values,
             int64_t values_capacity, int32_t *mask_words, uint8_t *mask_bool, void *stream);

/* Per-piece slot mask of `acting` (device int8 N; NULL = current turn):
 * slots: device uint8 (N, 120, 80), 16-byte aligned; slots[i][pid][s] = 1 iff
 * piece pid can take slot s. Slots 0-3 road steps (+x,-x,+y,-y), 4-7 camp
 * diagonals, 8-55 a non-engineer's straight rail runs (8 + dir*12 + k), 56-67
 * its curve-rail destinations, an engineer's rail destinations from slot 8;
 * the two BFS sections are packed from their first slot. Each piece row holds
 * as many ones as that piece has legal moves. Replaces legal_action_mask_batch
 * (bindings.cpp:951-990, game_state.cu:1964-2197; gpu_world.py:208-217,
 * gpu_rollout.py:862-869). */
int jq_legal_slots(jq_env *env, const int8_t *acting, uint8_t *slots, void *stream);

/* Observation of `observer` (device int8 N; NULL = current turn) in that seat's
 * canonical frame. fmt JQ_OBS_*; spatial: device (N,317,17,17) of the format's
 * element type; global: device float (N,28). JQ_OBS_U8 writes value codes
 * (jq_obs_decode_table maps them to the float32 values) and leaves the six
 * continuous planes zero; `aux` (device, 16-byte aligned, JQ_AUX_BYTES per row;
 * NULL to skip; NULL for the other formats) carries them: bytes 0-7 the float32
 * values of turn-history planes 64 and 65 (each constant over its plane), then
 * uint16 codes [4][289] of recency planes 253-256 per canonical cell, 0 for 0.0
 * and c > 0 for recency_table[plane - 253][c - 1] (jq_upload_recency's table,
 * exp(-(c - 1) / tau)). all_seats != 0 writes (N,4,...) rows; then
 * `observer` is an optional device int8 (N,4) observer map (slot k of env i
 * observes seat observer[i*4+k]; NULL = seat k), as upload_observer_seats sets
 * it (junqi_rl/gpu_rollout.py:983-1001). Replaces build_observation_single_seat /
 * build_observation_batch_resident (observation.cu:648-802). */
int jq_observe(jq_env *env, const int8_t *observer, int32_t fmt, int32_t all_seats, void *spatial,
               void *aux, float *global, void *stream);

/* Uploaded beliefs: copy (N, 4, 12, 289) float32 world-cell beliefs per (env,
 * observer) into the handle (from host memory if from_host, else from device
 * memory; the buffer is allocated on the first call) and make jq_observe read
 * its belief planes 12-23 and 27-50 from them: the observer's value at each
 * teammate / enemy piece's cell where > 0 (upload_beliefs,
 * junqi_rl/gpu_rollout.py:966-981; observation.cu:246-372). Globals keep the
 * BeliefTensor remaining counts. Such observations are JQ_OBS_F32 / JQ_OBS_BF16
 * only (arbitrary floats have no u8 code). jq_clear_beliefs returns to the
 * handle's own BeliefTensor beliefs. */
int jq_upload_beliefs(jq_env *env, const void *beliefs, int32_t from_host, void *stream);
int jq_clear_beliefs(jq_env *env);

/* Kernel timing of the observation (instrumentation; no counterpart in the
 * reference). While jq_obs_timing(env, 1) is in force, every observation launch
 * of the handle (jq_observe and the observation inside jq_env_step) is
 * bracketed by a pair of HIP events on the launch's stream; jq_obs_timing(env,
 * 0) pauses that. jq_obs_timing_read waits for the launches recorded since the
 * last read and returns their summed kernel time and count; at most
 * JQ_OBS_TIMING_MAX launches are recorded between two reads. */
#define JQ_OBS_TIMING_MAX 65536
int jq_obs_timing(jq_env *env, int32_t enable);
int jq_obs_timing_read(jq_env *env, double *total_ms, int64_t *launches);

/* The 256-entry float32 decode table of JQ_OBS_U8 codes (host pointer out). */
int jq_obs_decode_table(float *host_out256);

/* Samplers over the CSR jq_legal / jq_env_step wrote for the current state
 * (values_capacity as given there; a row that does not lie inside it, or an
 * empty row, gives -1). Counter-based Philox4x32-10 (Salmon et al., SC'11),
 * key (seed lo, seed hi):
 * jq_sample_uniform: index = (u * count) >> 32, u = word 0 of counter
 *   (env, ply lo, ply hi, 0); the world id values[offsets[env] + index].
 * jq_sample_logits: every canonical id c of the acting seat (`acting`, device
 *   int8 N; NULL = current turn) carries the logit z_c = Phi^-1((u_c + 1/2) / 2^32),
 *   u_c = word 0 of counter (env, ply lo, ply hi, 1 + c), i.i.d. N(0,1); the
 *   pick is the argmax of z over the legal ids (ties to the lowest c, as
 *   torch.argmax), computed exactly as the argmax of u_c. The reference's
 *   random opponent is this argmax with Gumbel noise over the legal mask
 *   (junqi_rl/training/gpu_collector.py:799-810). actions_out gets the world id,
 *   canonical_out (may be NULL) the canonical id. */
int jq_sample_uniform(jq_env *env, const int32_t *counts, const int32_t *offsets, const int32_t *values,
                      int64_t values_capacity, uint64_t seed, uint64_t ply, int32_t *actions_out, void *stream);
int jq_sample_logits(jq_env *env, const int8_t *acting, const int32_t *counts, const int32_t *offsets,
                     const int32_t *values, int64_t values_capacity, uint64_t seed, uint64_t ply,
                     int32_t *actions_out, int32_t *canonical_out, void *stream);

/* One fused env-step for the whole batch: sample with `sampler` (JQ_SAMPLE_*,
 * from the CSR of the previous call, if actions == NULL) -> step -> auto-reset
 * terminated envs from the pool -> legal (counts/offsets/values/mask) ->
 * observation of the new acting seat. Buffers and values_capacity as in the
 * calls above (with a small capacity the step is applied, counts / offsets /
 * mask are written and JQ_E_CAPACITY comes back before values and the
 * observation). hash: device uint64 (N), each env's Zobrist hash after its ply
 * and before any restart; terminated / reward as jq_step's; actions_out the
 * action taken (world id, -1 none).
 * With a u8 observation, values_capacity >= N * JQ_MAX_LEGAL and N <= 671,088 the CSR pass,
 * which then also writes the canonical mask words, runs on a library-owned
 * side stream beside the observation (they share no data); `stream` waits for
 * it before the call's work counts as done, so the call stays ordered on
 * `stream` like any other.
 * Sampling reads the rows the previous jq_env_step / jq_legal call wrote into
 * counts / offsets / values: after jq_reset_seeded, jq_reset_lineups or
 * jq_reset_terminated those rows describe the old positions, so call jq_legal
 * (or pass actions) before the next sampled step. A stale id that is not legal
 * in the new position is rejected like any illegal action (that env does not
 * move); reads stay inside values_capacity. */
int jq_env_step(jq_env *env, const int32_t *actions, int32_t sampler, uint64_t sample_seed, uint64_t ply,
                int64_t reset_seed, int32_t *counts, int32_t *offsets, int32_t *values, int64_t values_capacity,
                int32_t *mask_words, int32_t obs_fmt, void *spatial, void *aux, float *global,
                uint8_t *terminated, float *reward, uint64_t *hash, int32_t *actions_out, void *stream);

/* State import / export (host memory), one field at a time. Replaces
 * DeviceGameStateBatch.copy_to_host / copy_from_host (bindings.cpp:73-198).
 * jq_field_info gives the per-env element count and element size of a field. */
enum jq_field {
    JQ_F_CELL = 0,        /* int8  [289]   pid on the cell, -1 empty */
    JQ_F_PTYPE = 1,       /* int8  [128]   PieceType per pid (-1 absent) */
    JQ_F_POS = 2,         /* int16 [128]   flat cell, -1 dead/absent */
    JQ_F_ZERO = 3,        /* int16 [128]   initial cell, -1 none */
    JQ_F_MOVE_COUNT = 4,  /* int16 [128] */
    JQ_F_ACTIVE_EAT = 5,  /* int16 [128] */
    JQ_F_PASSIVE_SURV = 6,/* int16 [128] */
    JQ_F_DEATH_REASON = 7,/* int8  [128]  -1 alive */
    JQ_F_DEATH_STEP = 8,  /* int16 [128] */
    JQ_F_DEATH_LOC = 9,   /* int16 [128] */
    JQ_F_BELIEF = 10,     /* uint8 [4][128] belief row code per observer */
    JQ_F_REMAINING = 11,  /* int8  [4][4][12] */
    JQ_F_REM_TRACKED = 12,/* uint8 [4] bit s = remaining[s] tracked */
    JQ_F_CM_DIRECT_LO = 13, JQ_F_CM_DIRECT_HI = 14, JQ_F_CM_DIRECT_TYPE = 15,
    JQ_F_CM_LAST_DIRECT = 16, JQ_F_CM_OTHER_COUNT = 17, JQ_F_CM_CHAIN_LO = 18,
    JQ_F_CM_CHAIN_HI = 19, JQ_F_CM_CHAIN_TYPE = 20, JQ_F_CM_LAST_CHAIN = 21,
    JQ_F_CM_EATEN_LO = 22, JQ_F_CM_EATEN_HI = 23, JQ_F_CM_FLOOR = 24,
    JQ_F_CM_FLOOR_STEP = 25,
    JQ_F_CM_FLAGS = 26,   /* uint8 [4][128] bit0 is_gongb, bit1 not_gongb, bit2 attacked_by_known_gongb */
    JQ_F_HIST = 27,       /* int32 [32] ring of src | dst<<16 */
    JQ_F_HIST_META = 28,  /* int32 [1] count | head<<8 */
    JQ_F_TURN = 29,       /* int8 */
    JQ_F_TERMINATED = 30, /* uint8 */
    JQ_F_WINNER = 31,     /* int8 -1/0/1 */
    JQ_F_DRAW = 32,       /* uint8 */
    JQ_F_SEAT_DEAD = 33,  /* uint8 bitmask */
    JQ_F_FLAG_REV = 34,   /* uint8 bitmask */
    JQ_F_MOVE_COUNTER = 35, /* int32 */
    JQ_F_MSLC = 36,       /* int32 moves since last combat */
    JQ_F_ZOBRIST = 37,    /* uint64 */
    JQ_F_COUNT = 38
};
int jq_field_info(int32_t field, int32_t *elems_per_env, int32_t *elem_bytes);
int jq_get_field(jq_env *env, int32_t field, void *host_dst);
int jq_set_field(jq_env *env, int32_t field, const void *host_src);
/* Device address of element 0 of a state field and its strides in bytes between
 * envs and between a field's elements (zero-copy strided views, e.g. turn_torch:
 * junqi_rl/gpu_rollout.py:1159-1193). Fields live inside per-piece, per-observer
 * and per-env records, so the strides are generally larger than the element. */
int jq_field_ptr(jq_env *env, int32_t field, void **dev_ptr, int64_t *env_stride, int64_t *elem_stride);
/* After jq_set_field edits: recompute every env's Zobrist hash and re-seed the
 * four beliefs from the current board (GameState.__post_init__, state.py:346-483;
 * BeliefTensor.initial, info_model.py:218-265). Also rebuilds the compact
 * combat-memory summaries the observation reads, so edits of JQ_F_CM_* fields
 * (through jq_set_field or a jq_field_ptr view) reach observations only after
 * this call or jq_rehash. */
int jq_finalize_import(jq_env *env, void *stream);
/* jq_finalize_import restricted to the envs whose env_mask (device uint8, N)
 * entry is nonzero; the others keep their hash, beliefs and summaries.
 * Synchronises. */
int jq_finalize_import_masked(jq_env *env, const uint8_t *env_mask, void *stream);
/* Recompute every env's Zobrist hash and combat-memory summaries from its
 * current fields (after editing scalar fields such as the termination flags);
 * beliefs are left as they are. */
int jq_rehash(jq_env *env, void *stream);

/* ---- compact rollout history ------------------------------------------------
 * Pre-action state of every env at each of num_steps rollout steps (row
 * step * num_envs + env), from which PPO minibatches are rebuilt: observations
 * and canonical legal masks are recomputed for the requested rows instead of
 * being stored. Every per-env block is kept (board, pieces, all four observers'
 * combat memory and belief codes, remaining counts, counters, move ring):
 * jq_history_bytes() = num_steps * num_envs * 35972 bytes. Replaces
 * junqi_cuda.DeviceRolloutHistory (src/env/cuda/src/rollout_history.cu:160-525)
 * behind GpuRolloutHistory (junqi_rl/gpu_rollout.py:107-217). */
typedef struct jq_history jq_history;
int jq_history_create(jq_history **out, int32_t num_envs, int32_t num_steps, int32_t show_mode, int32_t device);
int jq_history_destroy(jq_history *hist);
int jq_history_bytes(const jq_history *hist, int64_t *bytes);
/* Copy env's current state into row block `step` (DeviceRolloutHistory::snapshot,
 * rollout_history.cu:190-287). `acting` (device int8, N) is accepted for the
 * reference's signature; all observers' beliefs are stored, so it is not read.
 * env must have num_envs games, the history's show mode and device. */
int jq_history_snapshot(jq_history *hist, jq_env *env, const int8_t *acting, int32_t step, void *stream);
/* Rebuild `batch` rows: flat (device int64, batch) row indices, observer (device
 * int8, batch) the seat each row is observed and masked for. Writes spatial /
 * aux / global like jq_observe (fmt JQ_OBS_*), and the canonical legal mask of
 * the observer seat as mask_words (device int32 (batch, 521)) and/or mask_bool
 * (device uint8 (batch, 16641)); any output may be NULL. Rows outside
 * [0, num_steps * num_envs) are rebuilt from the empty terminated state.
 * (DeviceRolloutHistory::reconstruct, rollout_history.cu:289-523.) Internal
 * scratch of `batch` rows is kept between calls (grown when needed), so calls
 * on one history must not overlap on different streams. */
int jq_history_reconstruct(jq_history *hist, const int64_t *flat, const int8_t *observer, int32_t batch, int32_t fmt,
                           void *spatial, void *aux, float *global, int32_t *mask_words, uint8_t *mask_bool,
                           void *stream);

/* The same rebuild with no device allocation: for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The rebuilt rows live in one
 * file-scope device array of the library, JQ_NOALLOC_MAX_ROWS rows (21.45 MB,
 * held on each device the library runs on until the process ends), shared by
 * every call on that device: calls that overlap on one device race, so keep
 * them on one stream or serialise them. batch > JQ_NOALLOC_MAX_ROWS returns
 * JQ_E_ARG; split larger minibatches. Outputs equal jq_history_reconstruct's. */
#define JQ_NOALLOC_MAX_ROWS 1024
int jq_history_reconstruct_noalloc(jq_history *hist, const int64_t *flat, const int8_t *observer, int32_t batch,
                                   int32_t fmt, void *spatial, void *aux, float *global, int32_t *mask_words,
                                   uint8_t *mask_bool, void *stream);

/* ---- legal-support storage: dense mask rows <-> id lists ----------------------
 * Rollout buffers keep each transition's legal support as ids
 * (junqi_rl/training/rollout_gpu.py:119-198). jq_mask_count: counts (device
 * int32, n) = nonzero bytes of each row of a dense (n, d) uint8 mask.
 * jq_mask_to_ids: ids (device int32, (n, k_max)) = each row's nonzero columns in
 * order, then zeros; every count must be <= k_max (check jq_mask_count first:
 * _dense_mask_to_csr raises before it writes, rollout_gpu.py:119-167).
 * jq_ids_to_mask: out (device uint8, (batch, d)) = rows idx (device int64,
 * batch) of the (rows, k_max) id lists with their counts as dense rows; ids
 * outside [0, d) and rows outside [0, rows) leave zeros
 * (_csr_to_dense_selected, rollout_gpu.py:170-198). Launched on the current
 * device. */
int jq_mask_count(const uint8_t *mask, int32_t n, int32_t d, int32_t *counts, void *stream);
int jq_mask_to_ids(const uint8_t *mask, int32_t n, int32_t d, int32_t k_max, int32_t *ids, void *stream);
int jq_ids_to_mask(const int32_t *ids, const int32_t *counts, int64_t rows, int32_t k_max, const int64_t *idx,
                   int32_t batch, int32_t d, uint8_t *out, void *stream);

/* Synchronise `stream`. */
int jq_sync(void *stream);

#ifdef __cplusplus
}
#endif
#endif
