// Host-built constant tables of the 17x17 Junqi board, uploaded once per device.
//
// Derived from the board's closed forms: seat rectangles, camps, strongholds,
// the rail ring of each seat, the nine-grid with its two-step links and the four
// corner arcs (reference junqi_core/board.py:88-279, rail_topology.py:60-276,
// _movegen_tables.py:155-467). Layouts are chosen for the device: rail cells are
// re-indexed 0..72 so an engineer's reachable set fits two 64-bit ballots.
#pragma once
#include <cstdint>

namespace jq {

constexpr int NC = 289;
constexpr int NONB = 129;
constexpr int NRAIL = 73;
constexpr int NP = 120;

// cell flag bits
enum : uint16_t {
    CF_ON = 1u << 0, CF_RAIL = 1u << 1, CF_CAMP = 1u << 2, CF_SH = 1u << 3,
    CF_NG = 1u << 4, CF_ARC = 1u << 5,
};

struct Tables {
    uint16_t cflags[NC];          // CF_* | curve_id << 8
    int16_t adj[NC][4];           // +x,-x,+y,-y on-board neighbours, -1 none
    int16_t diag[NC][4];          // diagonal neighbours with a camp endpoint, -1 none
    int8_t railidx[NC];           // rail index 0..72 or -1
    int16_t railcell[NRAIL];      // rail index -> flat
    uint64_t rnbr[NRAIL][2];      // rail-graph neighbour set as a 73-bit mask
    int16_t rays[NRAIL][4][12];   // straight rail runs per direction (-1 pad)
    int8_t raylen[NRAIL][4];
    int16_t crays[NRAIL][2][11];  // curve-rail chain runs both ways (-1 pad)
    int8_t craylen[NRAIL][2];
    int16_t f2c[NC];              // flat -> compact (-1 off board)
    int16_t c2f[NONB];
    int16_t rot[4][NC];           // world flat -> canonical flat of observer s
    int16_t unrot[4][NC];         // canonical flat -> world flat
    uint8_t rotc[4][NONB];        // world compact -> canonical compact
    int16_t home[NP];             // pid -> initial flat (-1 for camp slots)
    int8_t slotch[30];            // seat slot -> piece_slot plane (-1 camps)
    uint8_t statics[NC];          // board_static planes 0..4 as bits
    int16_t sh_other[NC];         // stronghold cell -> the other stronghold of that seat
    int8_t owner[NC];             // owning seat or -1
    int8_t localidx[NC];          // slot index in the owner's rectangle or -1
    // compact-cell forms for bitboard move generation (129-bit sets, bit c =
    // compact cell c; compact order is flat order, so a straight run's cells
    // rise (+x, +y) or fall (-x, -y) in compact index)
    alignas(8) uint8_t adjc[NONB][8];     // road neighbours then camp diagonals, compact (0xFF none)
    uint64_t adjm[NONB][2][3];            // adjc[c][4h .. 4h + 3] as a 129-bit set, h = 0, 1
    uint64_t raym[NRAIL][4][3];           // straight runs (+x, -x, +y, -y) as compact masks
    alignas(16) uint8_t crayc[NRAIL][2][16];  // curve runs in walk order, compact (0xFF pad)
    uint8_t railc[NRAIL];                 // rail index -> compact
    int8_t railidxc[NONB];                // compact -> rail index or -1
    uint64_t campm[3];                    // camp cells
    // 289-bit flat masks: a cell's compact index is the number of on-board
    // cells below it, its rail index the number of rail cells below it
    uint64_t onm[5], railm[5], shm[5];
    uint8_t canc[4][NC];          // world flat -> canonical compact of observer s (0xFF off board)
};

void build_tables(Tables &t);
void seat_cell(int seat, int slot, int &x, int &y);

// CPython random.Random(seed) lineup stream of junqi_core.setup.generate_random_setup
// (setup.py:162-258): four lineups of 30 piece types per seed.
void generate_setup(uint64_t seed, int8_t out[120]);
// pool_size setups from one random.Random(seed) stream (junqi_rl/gpu_rollout.py:255-275)
void generate_pool(uint64_t seed, int pool_size, int8_t *out);

// Canonical / mixed setup styles of junqi_rl/gpu_rollout.py:278-382 and 701-728.
enum { SETUP_CANONICAL = 1, SETUP_MIXED = 2 };
// style letter 'T', 'D', 'G', 'F' -> index into the canonical lineups, else -1
int canonical_style(char c);
// count setups; styles are canonical_style indices. per_game_seed: setup i from
// random.Random(seed + i) (GpuRollout.reset); else all from one random.Random(seed)
// stream (the pool builders).
void generate_styled(int mode, uint64_t seed, int count, bool per_game_seed, const int8_t *styles, int nstyles,
                     int8_t *out);

// validate_lineup (setup.py:60-136) of one seat's 30 slots: 0 when C1-C5 hold,
// else the LV_* bits of every rule broken (LV_TYPE alone for a value that is not
// a PieceType).
enum { LV_TYPE = 1, LV_C1 = 2, LV_C2 = 4, LV_C3 = 8, LV_C4 = 16, LV_C5 = 32 };
int validate_lineup(const int8_t *lineup30);

}  // namespace jq
