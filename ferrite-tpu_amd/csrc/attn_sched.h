// Work decomposition and LDS ring schedules of the causal attention kernels.
//
// The kernels in attention.hip take every block -> tile mapping, every split of a
// sweep and every "which tile goes into which ring slot at which step" decision
// from here, and so does the host-side schedule checker
// (tests/cpp/attn_schedule_test.cpp), which replays the launches over a sweep of
// shapes on the CPU: every output row written exactly once, no ring slot
// refilled while a wave may still read it, every tile landed (by the waits the
// kernels issue) before its first read. Plain integer functions, usable from
// host and device code.
#pragma once

#if defined(__HIPCC__) || defined(__HIP__)
#define FERRITE_SCHED __host__ __device__ constexpr
#else
#define FERRITE_SCHED constexpr
#endif

// Share (percent) of a pair's tiles that the older workgroup takes in the split
// forward, dK/dV and dQ kernels when two share a CU, and the fewest 128-row
// tiles for which the backward splits then; compile-time settings so that
// other values can be built and timed.
#ifndef FERRITE_FWD_OLDER_SHARE
#define FERRITE_FWD_OLDER_SHARE 70
#endif
#ifndef FERRITE_FWD_SPLIT_MIN_TWO
#define FERRITE_FWD_SPLIT_MIN_TWO 64
#endif
#ifndef FERRITE_DKV_OLDER_SHARE
#define FERRITE_DKV_OLDER_SHARE 62
#endif
#ifndef FERRITE_DQ_OLDER_SHARE
#define FERRITE_DQ_OLDER_SHARE 62
#endif
#ifndef FERRITE_BWD_SPLIT_MIN_TWO
#define FERRITE_BWD_SPLIT_MIN_TWO 32
#endif

namespace ferrite {
namespace sched {

// ---- grids -----------------------------------------------------------------
// A causal query-tile grid runs its heaviest (last) tiles first. zig (a grid
// resident all at once, two workgroups per CU): the second half of the grid
// takes the light tiles in rising order, so that block b and block b + grid / 2,
// which the dispatcher places on one CU, pair a long and a short sweep.
// blk = blockIdx / (B H); n = query tiles per head.
FERRITE_SCHED int query_tile(int blk, int n, bool zig) {
  return !zig || blk < n - n / 2 ? n - 1 - blk : blk - (n - n / 2);
}

// A causal key-block grid (dK/dV) runs its heaviest (first) blocks first; zig
// as above, the second half in falling order from the last block.
FERRITE_SCHED int key_block(int blk, int n, bool zig) {
  return !zig || blk < n - n / 2 ? blk : n - 1 - (blk - (n - n / 2));
}

// Wide head dims (D a multiple of 128 above 128 or 256): grid = heads x tiles x
// 128-column output slabs; block -> (head, tile, slab) with heads fastest, then
// tiles (heaviest causal tiles first where heavy_last: the query tiles of the
// forward and dQ; dK/dV's first key tiles are its heaviest), then slabs.
struct WideCoord {
  int bh, tile, slab;
};
FERRITE_SCHED WideCoord wide_coord(int block, int bh_count, int n_tiles, bool heavy_last) {
  const int rest = block / bh_count, t = rest % n_tiles;
  return WideCoord{block % bh_count, heavy_last ? n_tiles - 1 - t : t, rest / n_tiles};
}

// ---- the split long-context forward ---------------------------------------
// Key tiles [t0, t1) of query tile qt; role 0 / 1: block A's / B's share of a
// split tile (partial state, merged by the later of the two), -1: a whole tile.
struct Segment {
  int qt, t0, t1, role;
};
constexpr int kWholeTile = 0x7fffffff;  // t1 of a segment that runs to the tile's diagonal

// With 128-row query tiles (two 64-key tiles per query tile) and an even n,
// the tiles L = n - 1 - p and p of pair p hold 2 (L + 1) + 2 (p + 1) = 2 (n + 1)
// key tiles. Laid end to end (L's key tiles, then p's), they are cut after
// `cut` key tiles (0 < cut < 2 (n + 1)): block A of the pair (blk < n / 2) takes
// the tiles before the cut, block B (blk = p + n / 2) those after it. The tile
// the cut falls in (L if cut < 2 (L + 1), else p) is shared: its lower keys
// are A's (role 0), its upper keys B's (role 1). A cut at L's end shares none.
// Returns the number of segments (1 or 2) written to seg.
FERRITE_SCHED int split_segments(int blk, int n, int cut, Segment* seg) {
  const int half = n / 2, pair = blk % half, L = n - 1 - pair, nl = 2 * (L + 1);
  if (blk < half) {
    if (cut < nl) {
      seg[0] = Segment{L, 0, cut, 0};
      return 1;
    }
    seg[0] = Segment{L, 0, kWholeTile, -1};
    if (cut == nl) return 1;
    seg[1] = Segment{pair, 0, cut - nl, 0};
    return 2;
  }
  if (cut < nl) {
    seg[0] = Segment{L, cut, kWholeTile, 1};
    seg[1] = Segment{pair, 0, kWholeTile, -1};
    return 2;
  }
  seg[0] = Segment{pair, cut - nl, kWholeTile, cut == nl ? -1 : 1};
  return 1;
}

// Launch choices of the split kernels (128-row tiles) for B H = bh heads of S
// rows on a device of `cus` CUs. A split applies to a grid resident all at
// once (bh nq <= 2 CUs) with an even number nq of tiles, where it pays: with
// one workgroup per CU (bh nq <= CUs) from min_one tiles on, with two from
// min_two on (a shorter sweep gains less than the exchange of the shared tile
// costs; the causal, bf16, S % 128 == 0 and head-dim conditions are the
// caller's). With one workgroup per CU, A and B run at the same pace: equal
// halves. Two workgroups on a CU do not share it evenly: the older one (A,
// dispatched in the grid's first half) wins the issue ties, so A takes
// older_share percent of the pair's tiles.
struct SplitRule {
  int min_one, min_two, older_share;
};
constexpr int kSplitRows = 128;
// The forward: A runs about 2.5 stages for each of B's.
constexpr SplitRule kFwdSplit{16, FERRITE_FWD_SPLIT_MIN_TWO, FERRITE_FWD_OLDER_SHARE};
// dK/dV (key blocks sweeping query tiles) and dQ (query tiles sweeping key
// tiles) at head dims <= 64: A takes 62% (1x8x8192x64 on MI355X, shares 55 /
// 62 / 70 / 78: dK/dV 133.3 / 131.4 / 136.1 / 140.2 us against 157.1 unsplit,
// dQ with delta 105.9 / 105.2 / 105.8 / 107.6 against 116.1), and two
// workgroups per CU split from 32 tiles on (1x16x4096x64: dK/dV 87.9 -> 79.4,
// dQ 66.0 -> 63.5 us; 4x8x2048x64, 16 tiles: dQ 38.9 -> 41.3, dK/dV even).
constexpr SplitRule kDkvSplit{16, FERRITE_BWD_SPLIT_MIN_TWO, FERRITE_DKV_OLDER_SHARE};
constexpr SplitRule kDqSplit{16, FERRITE_BWD_SPLIT_MIN_TWO, FERRITE_DQ_OLDER_SHARE};
FERRITE_SCHED bool split_applies(long long bh, long long S, int cus, SplitRule r) {
  const long long nq = S / kSplitRows, grid = nq * bh;
  return S % kSplitRows == 0 && nq % 2 == 0 && grid <= 2LL * cus && nq >= (grid <= cus ? r.min_one : r.min_two);
}
FERRITE_SCHED int split_cut(long long bh, long long S, int cus, SplitRule r) {
  const long long nq = S / kSplitRows;
  return nq * bh <= cus ? (int)nq + 1 : (int)((2 * (nq + 1) * r.older_share + 50) / 100);
}
FERRITE_SCHED bool fwd_split_applies(long long bh, long long S, int cus) { return split_applies(bh, S, cus, kFwdSplit); }
FERRITE_SCHED int fwd_split_cut(long long bh, long long S, int cus) { return split_cut(bh, S, cus, kFwdSplit); }
// ZIG (query_tile, key_block) for a grid of `grid` workgroups that admits
// `per_cu` workgroups per CU: when all of them are resident at once.
FERRITE_SCHED bool resident(long long grid, int per_cu, int cus) { return grid <= (long long)per_cu * cus; }

// ---- rings -------------------------------------------------------------------
// Forward (attn_fwd_sw_kernel), SLOTS = 3 (D <= 128) or 2 (D = 256, whose
// 64-key K and V tiles take 68 KB a slot), tile t in slot t % SLOTS. Stage j
// (-1 .. n) reads K_{j+1} (S products) and V_{j-1} (P V products).
// Three slots: the prologue loads K_0 and K_1; stage j loads K_{j+3} and
// V_{j+1} after its barrier; before the barrier of stage j >= 0 a wave lets its
// previous stage's loads (2 kDma instructions) stay in flight, before stage -1
// its K_1 (kDma). Two slots: the prologue loads K_0; stage j loads K_{j+2} and
// V_j (none at stage -1); a wave lets nothing stay in flight before a barrier.
constexpr int kFwdSlots = 3;
FERRITE_SCHED int fwd_k_loaded(int j, int slots = kFwdSlots) { return j + slots; }
FERRITE_SCHED int fwd_v_loaded(int j, int slots = kFwdSlots) { return j + slots - 2; }
FERRITE_SCHED bool fwd_v_loads(int j, int slots = kFwdSlots) { return fwd_v_loaded(j, slots) >= 0; }
FERRITE_SCHED int fwd_k_read(int j) { return j + 1; }
FERRITE_SCHED int fwd_v_read(int j) { return j - 1; }
FERRITE_SCHED int fwd_prologue_k(int slots = kFwdSlots) { return slots - 1; }  // K tiles the prologue loads
FERRITE_SCHED int fwd_in_flight(int j, int kdma, int slots = kFwdSlots) {
  return slots == 2 ? 0 : j >= 0 ? 2 * kdma : kdma;
}

// dQ (attn_dq_pp_kernel), SLOTS = 2 or 3, tile t in slot t % SLOTS. The
// prologue loads tiles 0 .. SLOTS - 2; after the barrier of step t the wave
// loads tile t + SLOTS - 1 (if any) and reads tile t. Before that barrier a
// wave lets tile t + 1 stay in flight (three slots) or nothing.
FERRITE_SCHED int dq_loaded(int t, int slots) { return t + slots - 1; }
FERRITE_SCHED int dq_in_flight(int t, int n, int slots, int ops_per_tile) {
  return slots == 3 && t + 1 < n ? ops_per_tile : 0;
}

// dK/dV at D = 64 (attn_dkv_sw_kernel), four slots, query tile t in slot t % 4,
// half-steps h = -1 .. 2 nt (two per 64-query tile). The prologue loads tiles 0
// and 1; half-step h loads half of tile (h + 5) / 2's instructions (the first
// half in odd half-steps) and reads tiles (h - 1) / 2 .. (h + 1) / 2
// (arithmetic shifts). A barrier opens every odd half-step; before it a wave
// lets one tile's instructions stay in flight.
constexpr int kDkvSwSlots = 4;
FERRITE_SCHED int dkv_sw_loaded(int h) { return (h + 5) >> 1; }
FERRITE_SCHED int dkv_sw_first_read(int h) { return (h - 1) >> 1; }
FERRITE_SCHED int dkv_sw_last_read(int h) { return (h + 1) >> 1; }

// dK/dV at D = 128 (attn_dkv_rs_kernel), three slots, query tile t in slot
// t % 3, half-steps h = -1 .. 2 nt. The prologue loads tile 0; odd half-step h
// loads tile (h + 3) / 2, and tile t is read in half-steps 2 t - 1 .. 2 t + 2.
// A barrier opens every half-step; before an odd one a wave waits for all its
// loads.
constexpr int kDkvRsSlots = 3;
FERRITE_SCHED int dkv_rs_loaded(int h) { return (h & 1) ? (h + 3) >> 1 : -1; }
FERRITE_SCHED int dkv_rs_first_read(int t) { return 2 * t - 1; }
FERRITE_SCHED int dkv_rs_last_read(int t) { return 2 * t + 2; }

// dK/dV at D = 256 in one pass (attn_dkv_q256_kernel), steps h = -1 .. nh + 1
// over 32-query granules x = 0 .. nh - 1: Q (and lse) of granule x in Q slot
// x % 5, dO (and delta) in dO slot x % 3; the prologue loads Q 0, step h loads
// Q h + 2 and dO h + 1 (by the light waves) after its barrier, and a wave waits
// for all its loads before every barrier. Q x is read in steps x - 1 (S, role
// A), x + 1 (dK, role B) and x + 2 (dK, role B'), lse x in step x; dO x in
// steps x (dP, role B) and x + 1 (dV, roles A and A'), delta x in step x + 1.
// P of granule x (role A, step x) is read by B and A' in step x + 1; dS of x
// (role B, step x + 1) by B' in step x + 2.
constexpr int kDkv256qQSlots = 5, kDkv256qDoSlots = 3;
FERRITE_SCHED int dkv256q_q_loaded(int h) { return h + 2; }
FERRITE_SCHED int dkv256q_do_loaded(int h) { return h + 1; }

}  // namespace sched
}  // namespace ferrite
