// Host-side replay of the causal attention kernels' schedules
// (ferrite-tpu_amd/csrc/attention.hip), over a sweep of shapes, with the grid
// orders, splits, launch choices and ring schedules taken from the kernels'
// own header (csrc/attn_sched.h). What each kernel does per step is restated
// here from attention.hip, kernel by kernel:
//
//   attn_fwd_sw_kernel   the forward (D = 128: 8 waves of 32 rows; D <= 64: 8
//                        waves, pairs splitting every key tile; the split
//                        long-context grid)
//   attn_dq_pp_kernel    dQ (D = 128: 4 waves, 2 slots; D = 64: 4 waves and 2
//                        slots, or 8 waves splitting every key tile on a
//                        resident grid; the split long-context grid)
//   attn_dkv_sw_kernel   dK/dV at D = 64 (4 waves, 4 slots, half-steps; the
//                        split long-context grid)
//   attn_dkv_rs_kernel   dK/dV at D = 128 (8 waves in two roles, 3 slots)
//   attn_dkv_q256_kernel dK/dV at D = 256 in one pass (four roles, a Q ring of
//                        5 and a dO ring of 3 granules, P and dS buffers)
//   attn_*_wide_kernel   head dims above 128 / 256 (the grid only: their LDS
//                        staging is synchronous, between two barriers)
//
// and checked:
//   * every output row (query rows for O and dQ, key rows for dK and dV) is
//     written exactly once; with a split, every key tile of every query tile
//     (every query tile of every key block) is swept exactly once, by shares
//     that one merge combines;
//   * every LDS ring read finds the tile it expects, loaded at an earlier step
//     and guaranteed complete by the wait counts each wave issues before the
//     barrier of the reading step;
//   * no load (a past-the-end tile's zero fill included) lands in a region
//     in the epoch of a read of it, or before a read of its previous contents.
#include "../../ferrite-tpu_amd/csrc/attn_sched.h"

#include <algorithm>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

using namespace ferrite::sched;

static int failures = 0;
static bool quiet = false;  // while planted mistakes run
static void fail(const std::string& what) {
  if (failures < 20 && !quiet) std::fprintf(stderr, "FAIL: %s\n", what.c_str());
  ++failures;
}

// ---------------------------------------------------------------------------
// One workgroup's LDS traffic. Time is counted in barrier epochs: epoch e runs
// from barrier e to barrier e + 1. Regions are small integers (ring slots and
// staging areas); a load covers one or more regions.
// ---------------------------------------------------------------------------
struct Part {
  int wave, seq;  // the wave's seq-th VMEM instruction
};
struct Load {
  int epoch;
  std::vector<int> regions;
  long label;
  std::vector<Part> parts;
};
struct Read {
  int epoch, region, wave;
  long label;
};

class Workgroup {
 public:
  Workgroup(int waves, const std::string& name) : waves_(waves), issued_(waves, 0), name_(name) {}
  int epoch() const { return epoch_; }
  // A barrier, before which wave w waits until at most in_flight[w] of its
  // VMEM instructions are outstanding (-1: no wait).
  void barrier(const std::vector<int>& in_flight) {
    ++epoch_;
    std::vector<int> done(waves_);
    for (int w = 0; w < waves_; ++w) {
      int c = complete_.empty() ? 0 : complete_.back()[w];
      if (in_flight[w] >= 0) c = std::max(c, issued_[w] - in_flight[w]);
      done[w] = c;
    }
    complete_.push_back(done);  // complete_[e - 1]: instructions done by barrier e
  }
  void barrier_all(int in_flight) { barrier(std::vector<int>(waves_, in_flight)); }
  // Wave w issues n instructions of the load (regions, label) in this epoch.
  void issue(int w, const std::vector<int>& regions, long label, int n) {
    Load* ld = nullptr;
    for (auto it = loads_.rbegin(); it != loads_.rend() && it->epoch == epoch_; ++it)
      if (it->label == label && it->regions == regions) ld = &*it;
    if (!ld) {
      loads_.push_back(Load{epoch_, regions, label, {}});
      ld = &loads_.back();
    }
    for (int i = 0; i < n; ++i) ld->parts.push_back(Part{w, issued_[w]++});
  }
  void read(int w, int region, long label) { reads_.push_back(Read{epoch_, region, w, label}); }
  // An instruction with no LDS side that still counts in the wave's VMEM counter (a store).
  void vmem(int w, int n) { issued_[w] += n; }

  // Every read finds its tile: the last load into the region up to and
  // including the read's epoch is that tile's, was issued in an earlier epoch
  // (a load in the read's own epoch would land while the read runs), and every
  // wave's part of it was waited for before the barrier that opened the read's
  // epoch. A region is therefore never refilled while a wave may still read it.
  void check() {
    for (const Read& r : reads_) {
      const Load* last = nullptr;
      for (const Load& l : loads_)
        if (l.epoch <= r.epoch && std::count(l.regions.begin(), l.regions.end(), r.region)) last = &l;
      if (!last || last->label != r.label || last->epoch == r.epoch) {
        fail(name_ + ": wave " + std::to_string(r.wave) + " reads region " + std::to_string(r.region) + " for " +
             std::to_string(r.label) + " in epoch " + std::to_string(r.epoch) + " but the last load into it is " +
             (last ? std::to_string(last->label) + " in epoch " + std::to_string(last->epoch) : std::string("none")));
        continue;
      }
      for (const Part& p : last->parts) {
        const int done = r.epoch >= 1 && r.epoch - 1 < (int)complete_.size() ? complete_[r.epoch - 1][p.wave] : 0;
        if (p.seq >= done) {
          fail(name_ + ": label " + std::to_string(r.label) + " read in epoch " + std::to_string(r.epoch) +
               " before wave " + std::to_string(p.wave) + "'s part of it is waited for");
          break;
        }
      }
    }
  }

 private:
  int waves_, epoch_ = 0;
  std::vector<int> issued_;
  std::vector<std::vector<int>> complete_;
  std::vector<Load> loads_;
  std::vector<Read> reads_;
  std::string name_;
};

// Row coverage of one output: counts[row] over the whole grid.
struct Coverage {
  std::vector<int> count;
  explicit Coverage(long rows) : count(rows, 0) {}
  void add(long r0, long n, long limit) {
    for (long r = r0; r < r0 + n && r < limit; ++r) ++count[r];
  }
  void expect_once(const std::string& name) {
    for (size_t r = 0; r < count.size(); ++r)
      if (count[r] != 1) {
        fail(name + ": row " + std::to_string(r) + " written " + std::to_string(count[r]) + " times");
        return;
      }
  }
};

constexpr int kCus = 256;

// Planted mistakes, to show that the checks catch them (main runs each on a few
// shapes and expects failures): 0 = the kernels' schedules.
static int g_mutation = 0;
static int k_loaded(int j, int slots) { return g_mutation == 1 ? j + slots - 1 : fwd_k_loaded(j, slots); }  // K a stage late
static int v_loaded(int j, int slots) { return g_mutation == 2 ? j + slots - 1 : fwd_v_loaded(j, slots); }  // V into a slot in use
static int fwd_wait(int j, int kdma, int slots) {
  return g_mutation == 3 ? fwd_in_flight(j, kdma, slots) + kdma : fwd_in_flight(j, kdma, slots);  // waits too shallow
}
static int dq_next(int t, int slots) { return g_mutation == 4 ? t + slots : dq_loaded(t, slots); }
static bool fwd_writes(int kh, int role) { return g_mutation == 5 ? role != 0 : kh == 0 && (role < 0 || role == 1); }
static int rs_loaded(int h) { return g_mutation == 6 ? ((h & 1) ? (h + 5) >> 1 : -1) : dkv_rs_loaded(h); }
static int q256q_loaded(int h) { return g_mutation == 9 ? h + 3 : dkv256q_q_loaded(h); }   // Q into a slot in use
static int do256q_loaded(int h) { return g_mutation == 10 ? h + 2 : dkv256q_do_loaded(h); }  // dO into a slot in use
// The half-step in which wave 0 of attn_dkv_rs_kernel writes tile t's scaled lse row (2t - 1).
static int rs_lse_write(int t) { return g_mutation == 11 ? 2 * t : 2 * t - 1; }  // a half-step late
constexpr int BK = 64;  // keys per tile of the forward and dQ rings, queries per tile of dK/dV's

// ---------------------------------------------------------------------------
// Forward: attn_fwd_sw_kernel. Regions 0 .. slots - 1: K slots, then the V
// slots (three of each at D <= 128, two at D = 256). Q rows are staged in the
// K slots past the prologue's tiles and in the V slots (d == D) and read
// between sync(-1) and a second barrier.
// ---------------------------------------------------------------------------
struct FwdCfg {
  int D, W, ksplit;
  bool zig, split;
};

// n, n_w of a wave in segment [t0, t1) of query tile qt (the kernel's segment()).
static void fwd_counts(const FwdCfg& c, int S, const Segment& sg, int wave, int& n, int& n_w, int& q0w, int& kh) {
  const int WR = c.W / c.ksplit, BQ = 32 * WR;
  const int wr = wave % WR;
  kh = wave / WR;
  q0w = sg.qt * BQ + 32 * wr;
  const int nfull = (std::min(sg.qt * BQ + BQ, S) - 1) / BK + 1;
  const int tt1 = std::min(sg.t1, nfull);
  n = tt1 - sg.t0;
  const int nwf = q0w < S ? (q0w + 31) / BK + 1 : 0;
  n_w = (kh == 1 && q0w % BK == 0 && sg.t0 == nwf - 1) ? 0 : std::max(std::min(nwf, tt1) - sg.t0, 0);
}

// The split's bookkeeping, per tile that a block sweeps (a query tile over key
// tiles, or a key block over query tiles): the ranges [t0, t1) its segments
// swept must cover [0, nfull(tile)) exactly once, and a shared tile must have
// exactly one share of each role.
typedef std::map<std::pair<int, int>, std::vector<std::pair<int, int>>> Swept;
typedef std::map<std::pair<int, int>, int> Roles;
template <typename NFull>
static void check_sweeps(const std::string& name, const Swept& swept, const Roles& roles, NFull nfull_of) {
  for (auto& kv : swept) {
    const int tile = kv.first.second;
    const int nfull = nfull_of(tile);
    std::vector<int> hits(nfull, 0);
    for (auto& r : kv.second)
      for (int t = r.first; t < r.second; ++t)
        if (t >= 0 && t < nfull) ++hits[t];
    for (int t = 0; t < nfull; ++t)
      if (hits[t] != 1) fail(name + ": tile " + std::to_string(tile) + " sub-tile " + std::to_string(t) + " swept " +
                             std::to_string(hits[t]) + " times");
  }
  for (auto& kv : roles)
    if (kv.second != 1) fail(name + ": more than one share of one role for tile " + std::to_string(kv.first.first));
  std::map<int, int> shared;
  for (auto& kv : roles) shared[kv.first.first] |= 1 << kv.first.second;
  for (auto& kv : shared)
    if (kv.second != 3) fail(name + ": tile " + std::to_string(kv.first) + " shared by one block only");
}

static void check_fwd(const FwdCfg& c, int bh, int S) {
  const int WR = c.W / c.ksplit, BQ = 32 * WR;
  const int nq = (S + BQ - 1) / BQ;
  const int slots = c.D > 128 ? 2 : 3;   // FwdW::kSlots
  const int kdma = c.D / 8 / c.W;        // K (or V) blocks per wave and tile: D / 8 blocks of 1 KB
  const int qdma = 32 * 2 * c.D / 1024;  // this wave's 32 Q rows, 1 KB per instruction
  const int cut = c.split ? fwd_split_cut(bh, S, kCus) : 0;
  const std::string name = "fwd D" + std::to_string(c.D) + (c.split ? " split" : c.zig ? " zig" : "") + " bh" +
                           std::to_string(bh) + " S" + std::to_string(S);
  Coverage rows((long)bh * S);
  // With the split: every (head, query tile) gets its key tiles from shares
  // that together sweep [0, nfull) once, and exactly one share per shared tile
  // of each role.
  Swept swept;
  Roles roles;
  for (int blk = 0; blk < nq; ++blk) {
    Segment seg[2];
    int nseg = 1;
    if (c.split)
      nseg = split_segments(blk, nq, cut, seg);
    else
      seg[0] = Segment{query_tile(blk, nq, c.zig), 0, kWholeTile, -1};
    // Every head runs the same schedule: simulate head 0, count rows for all.
    {
      const int h = 0;
      Workgroup wg(c.W, name + " blk" + std::to_string(blk));
      for (int sgi = 0; sgi < nseg; ++sgi) {
        const Segment& sg = seg[sgi];
        if (sgi > 0) wg.barrier_all(-1);  // the kernel's barrier between segments
        int n = 0, n_w[8], q0w[8], kh[8];
        for (int w = 0; w < c.W; ++w) fwd_counts(c, S, sg, w, n, n_w[w], q0w[w], kh[w]);
        const int nfull = (std::min(sg.qt * BQ + BQ, S) - 1) / BK + 1;
        if (h == 0) {
          swept[{0, sg.qt}].push_back({sg.t0, std::min(sg.t1, nfull)});
          if (sg.role >= 0) ++roles[{sg.qt, sg.role}];
        }
        // Labels: K tile t -> 1000 + t, V tile t -> 2000 + t, Q -> 3000 (per segment).
        const long base = 10000L * (sgi + 1);
        auto kslot = [&](int t) { return t % slots; };
        auto vslot = [&](int t) { return slots + t % slots; };
        // Prologue: K_0, this wave's Q rows, and with three slots K_1. The Q
        // rows take K slot 2 and the V slots (three slots), or K slot 1 and the
        // V slots (two: 16 KB a wave from K slot 1's start, wave 2 across
        // into V slot 0).
        const std::vector<int> qst = slots == 3 ? std::vector<int>{2, 3, 4, 5} : std::vector<int>{1, 2, 3};
        for (int w = 0; w < c.W; ++w) {
          wg.issue(w, {kslot(0)}, base + 1000, kdma);
          wg.issue(w, qst, base + 3000, qdma);
          if (fwd_prologue_k(slots) > 1) wg.issue(w, {kslot(1)}, base + 1001, kdma);
        }
        // sync(-1), the Q reads, a barrier.
        std::vector<int> fl(c.W, fwd_wait(-1, kdma, slots));
        wg.barrier(fl);
        for (int w = 0; w < c.W; ++w) {
          if (slots == 3) {
            wg.read(w, 2 + (w % 4), base + 3000);
          } else {
            if (w <= 2) wg.read(w, 1, base + 3000);
            if (w >= 2) wg.read(w, 2, base + 3000);
          }
        }
        wg.barrier_all(-1);
        // Stages -1 .. n: this wave's reads, then everyone's DMA.
        for (int j = -1; j <= n; ++j) {
          if (j >= 0) wg.barrier_all(fwd_wait(j, kdma, slots));
          for (int w = 0; w < c.W; ++w) {
            // K reads in stages -1 .. n_w - 2 (tile j + 1), V reads in 1 .. n_w (tile j - 1).
            if (n_w[w] > 0 && j <= n_w[w] - 2) wg.read(w, kslot(fwd_k_read(j)), base + 1000 + fwd_k_read(j));
            if (n_w[w] > 0 && j >= 1 && j <= n_w[w]) wg.read(w, vslot(fwd_v_read(j)), base + 2000 + fwd_v_read(j));
          }
          for (int w = 0; w < c.W; ++w) {
            wg.issue(w, {kslot(k_loaded(j, slots))}, base + 1000 + k_loaded(j, slots), kdma);
            // (Two slots: no V at stage -1; the kernel's instructions read nothing and still count.)
            if (fwd_v_loads(j, slots))
              wg.issue(w, {vslot(v_loaded(j, slots))}, base + 2000 + v_loaded(j, slots), kdma);
            else
              wg.vmem(w, kdma);
          }
        }
        // O rows: a whole tile's writers, or the merge of a shared one.
        for (int w = 0; w < c.W; ++w)
          if (q0w[w] < S && fwd_writes(kh[w], sg.role))
            for (int hh = 0; hh < bh; ++hh) rows.add((long)hh * S + q0w[w], 32, (long)hh * S + S);
      }
      wg.check();
    }
  }
  rows.expect_once(name + " O rows");
  check_sweeps(name, swept, roles, [&](int qt) { return (std::min(qt * BQ + BQ, S) - 1) / BK + 1; });
}

// ---------------------------------------------------------------------------
// dQ: attn_dq_pp_kernel. Tile t (K and V of 64 keys) in slot t % SLOTS.
// ---------------------------------------------------------------------------
struct DqCfg {
  int D, W, slots, ksplit;
  bool zig, split;
};

// The dQ rows a segment writes: a whole tile's, or a shared tile's once (by the
// second of its two blocks to arrive; counted here with role 0's share).
static bool dq_writes(int kh, int role) { return g_mutation == 7 ? (kh == 0) : (kh == 0 && role <= 0); }

static void check_dq(const DqCfg& c, int bh, int S) {
  const int BQ = 32 * c.W / c.ksplit;
  const int nq = (S + BQ - 1) / BQ;
  const int kdma = (c.D == 256 ? 32 : 16) / c.W;  // BwdTile: 16 (D = 256: 32) blocks per tile, split over the waves
  const int cut = c.split ? split_cut(bh, S, kCus, kDqSplit) : 0;
  const std::string name = "dq D" + std::to_string(c.D) + " W" + std::to_string(c.W) + (c.split ? " split" : "") +
                           " bh" + std::to_string(bh) + " S" + std::to_string(S);
  Coverage rows((long)bh * S);
  Swept swept;
  Roles roles;
  for (int blk = 0; blk < nq; ++blk) {
    Segment seg[2];
    int nseg = 1;
    if (c.split)
      nseg = split_segments(blk, nq, cut, seg);
    else
      seg[0] = Segment{query_tile(blk, nq, c.zig), 0, kWholeTile, -1};
    Workgroup wg(c.W, name + " blk" + std::to_string(blk));
    for (int sgi = 0; sgi < nseg; ++sgi) {
      const Segment& sg = seg[sgi];
      if (sgi > 0) wg.barrier_all(-1);  // the kernel's barrier between segments
      const int q0 = sg.qt * BQ;
      const int n_all = (std::min(q0 + BQ, S) - 1) / BK + 1;
      // The kernel's segment(): n tiles (key tiles t0 .. t0 + n - 1), n_w per wave.
      const int n = (sg.t1 == kWholeTile ? n_all : sg.t1) - sg.t0;
      swept[{0, sg.qt}].push_back({sg.t0, sg.t0 + n});
      if (sg.role >= 0) ++roles[{sg.qt, sg.role}];
      const long base = 10000L * (sgi + 1);
      int n_w[8], q0w[8], kh[8];
      for (int w = 0; w < c.W; ++w) {
        kh[w] = c.ksplit == 1 ? 0 : w / (c.W / c.ksplit);
        q0w[w] = q0 + 32 * (c.ksplit > 1 ? w % (c.W / c.ksplit) : c.W == 8 ? 2 * (w & 3) + (w >> 2) : w);
        const int nwf = q0w[w] < S ? std::min(q0w[w] + 31, S - 1) / BK + 1 : 0;
        n_w[w] = std::min(std::max(nwf - sg.t0, 0), n);
      }
      for (int t = 0; t < c.slots - 1 && t < n; ++t)
        for (int w = 0; w < c.W; ++w) wg.issue(w, {t % c.slots}, base + 1000 + t, 2 * kdma);
      for (int t = 0; t < n; ++t) {
        wg.barrier_all(dq_in_flight(t, n, c.slots, 2 * kdma));
        for (int w = 0; w < c.W; ++w)
          if (t < n_w[w]) wg.read(w, t % c.slots, base + 1000 + t);
        if (dq_next(t, c.slots) < n)
          for (int w = 0; w < c.W; ++w)
            wg.issue(w, {dq_next(t, c.slots) % c.slots}, base + 1000 + dq_next(t, c.slots), 2 * kdma);
      }
      for (int w = 0; w < c.W; ++w)
        if (q0w[w] < S && dq_writes(kh[w], sg.role))
          for (int hh = 0; hh < bh; ++hh) rows.add((long)hh * S + q0w[w], 32, (long)hh * S + S);
    }
    wg.check();
  }
  rows.expect_once(name + " dQ rows");
  check_sweeps(name, swept, roles, [&](int qt) { return (std::min(qt * BQ + BQ, S) - 1) / BK + 1; });
}

// ---------------------------------------------------------------------------
// dK/dV: key blocks of 128 rows sweep 64-query tiles from the diagonal on
// (a sweep of fewer than three tiles runs as three, the extra tiles reading as
// zeros). Regions: the ring slots; in attn_dkv_rs_kernel also the two P
// buffers (11, 12) that role A writes in half-step h and role B reads in h + 1,
// and each wave's K/V row staging (20 + w), which overlaps slot 2 and the P
// buffers.
// ---------------------------------------------------------------------------
static void check_dkv(int D, int bh, int S, bool zig, bool split = false) {
  const int BKV = 128, nk = (S + BKV - 1) / BKV;
  const bool rs = D == 128;
  const int W = rs ? 8 : 4, slots = rs ? kDkvRsSlots : kDkvSwSlots;
  const int kdma = (D == 64 ? 8 : 16) / W;     // Q (or dO) blocks per wave and tile
  const int cut = split ? split_cut(bh, S, kCus, kDkvSplit) : 0;
  const std::string name = std::string(rs ? "dkv_rs" : "dkv_sw") + (split ? " split" : zig ? " zig" : "") + " bh" +
                           std::to_string(bh) + " S" + std::to_string(S);
  Coverage krows((long)bh * S);
  Swept swept;
  Roles roles;
  for (int blk = 0; blk < nk; ++blk) {
    Segment seg[2];
    int nseg = 1;
    if (split)
      nseg = split_segments(blk, nk, cut, seg);
    else
      seg[0] = Segment{nk - 1 - key_block(blk, nk, zig), 0, kWholeTile, -1};
    Workgroup wg(W, name + " blk" + std::to_string(blk));
    for (int sgi = 0; sgi < nseg; ++sgi) {
      const Segment& sg = seg[sgi];
      if (sgi > 0) wg.barrier_all(-1);  // the kernel's barrier between segments
      // The kernel's segment(): key block kt = nk - 1 - qt over query tiles
      // first .. (the end of the queries, or the segment's end qlim).
      const int kt = nk - 1 - sg.qt;
      const int k0 = kt * BKV;
      const int first = k0 / BK + sg.t0;
      const int qlim = sg.t1 == kWholeTile ? S : (k0 / BK + sg.t1) * BK;
      const int nt = std::max((qlim + BK - 1) / BK - first, 3);
      const int nh = 2 * nt;
      swept[{0, kt}].push_back({sg.t0, (qlim + BK - 1) / BK - k0 / BK});
      if (sg.role >= 0) ++roles[{kt, sg.role}];
      const long sbase = 10000L * (sgi + 1) - 1000;
      {
      // Ops of one tile for wave w: Q and dO blocks, plus the statistics rows
      // (every wave in the one-role kernel; waves 0 and 4 in the role split).
      auto tile_ops = [&](int w) { return 2 * kdma + (rs ? ((w & 3) == 0 ? 1 : 0) : 2); };
      if (!rs) {
        for (int t = 0; t < 2; ++t)
          for (int w = 0; w < W; ++w) wg.issue(w, {t % slots}, sbase + 1000 + t, tile_ops(w));
        // Barriers before half-steps -1, 1, 3, ... (one tile's instructions may fly).
        for (int h = -1; h <= nh; ++h) {
          if (h & 1) {
            std::vector<int> fl(W);
            for (int w = 0; w < W; ++w) fl[w] = tile_ops(w);
            wg.barrier(fl);
          }
          for (int w = 0; w < W; ++w) {
            if (h <= nh - 2) wg.read(w, ((h + 1) >> 1) % slots, sbase + 1000 + ((h + 1) >> 1));  // S, dP of half h + 1
            if (h >= 0 && h <= nh - 1) wg.read(w, (h >> 1) % slots, sbase + 1000 + (h >> 1));  // P, dS of half h
            if (h >= 1) wg.read(w, ((h - 1) >> 1) % slots, sbase + 1000 + ((h - 1) >> 1));      // dV, dK of half h - 1
          }
          const int t = dkv_sw_loaded(h);
          for (int w = 0; w < W; ++w) {
            const int ops = tile_ops(w), firsthalf = ops / 2;
            wg.issue(w, {t % slots}, sbase + 1000 + t, (h & 1) ? firsthalf : ops - firsthalf);
          }
        }
      } else {
        // Prologue: tile 0, and each wave's K or V rows (8 KB) into the staging,
        // wave w at 8 w KB from slot 2's start: waves 0-3 inside slot 2 (35 KB),
        // wave 4 across its end and P buffer 0 (16 KB), waves 5-7 in the P
        // buffers. Region 20 + w is wave w's own piece.
        const std::vector<int> staging[8] = {{2, 20}, {2, 21}, {2, 22}, {2, 23},
                                             {2, 11, 24}, {11, 25}, {11, 12, 26}, {12, 27}};
        // Wave 0's statistics instruction loads the tile's lse row into registers (no LDS
        // region); it writes the row, scaled, into region 30 + t % slots at odd half-step
        // 2t - 1 (tile 0: -1), a ds_write modelled as an instant fill, and role A reads it
        // in the tile's two softmax half-steps.
        auto issue_tile = [&](int w, int t) {
          const int lse_reg = w == 0 ? 1 : 0;
          wg.issue(w, {t % slots}, sbase + 1000 + t, tile_ops(w) - lse_reg);
          wg.vmem(w, lse_reg);
        };
        for (int w = 0; w < W; ++w) {
          issue_tile(w, 0);
          wg.issue(w, staging[w], sbase + 3000 + w, 8);  // 32 rows of 256 bytes, 1 KB per instruction
        }
        for (int h = -1; h <= nh; ++h) {
          std::vector<int> fl(W, (h & 1) ? 0 : -1);
          wg.barrier(fl);
          if (h == -1)
            for (int w = 0; w < W; ++w) wg.read(w, 20 + w, sbase + 3000 + w);  // the rows back, in stage -1
          for (int t = std::max(h >> 1, 0); t <= ((h + 2) >> 1); ++t)
            if (rs_lse_write(t) == h) wg.issue(0, {30 + t % slots}, sbase + 7000 + t, 0);
          for (int w = 0; w < W; ++w) {
            for (int t = std::max((h - 1) >> 1, 0); t <= ((h + 1) >> 1) && t < nt; ++t)
              if (dkv_rs_first_read(t) <= h && h <= dkv_rs_last_read(t) && h <= nh) wg.read(w, t % slots, sbase + 1000 + t);
            // P of half h - 1 from A (written in half-step h - 1), read by B in h.
            if (w >= 4 && h >= 1) wg.read(w, 11 + ((h - 1) & 1), sbase + 5000 + h - 1);
            // The lse row of the half's tile, in role A's softmax.
            if (w < 4 && h >= 0 && h <= nh - 1) wg.read(w, 30 + (h >> 1) % slots, sbase + 7000 + (h >> 1));
          }
          const int t = rs_loaded(h);
          if (t >= 0)
            for (int w = 0; w < W; ++w) issue_tile(w, t);
          // A writes P of half h (ds_write, no VMEM count), modelled as an
          // instant fill of that buffer in this epoch.
          if (h >= 0 && h <= nh - 1)
            for (int w = 0; w < 4; ++w) wg.issue(w, {11 + (h & 1)}, sbase + 5000 + h, 0);
        }
      }
      }
      // dK/dV rows: a whole sweep's, or a shared block's once (by the second
      // of its two workgroups to arrive; counted with role 0's share).
      if (sg.role <= 0 || g_mutation == 8)
        for (int w = 0; w < (rs ? 4 : W); ++w)
          for (int hh = 0; hh < bh; ++hh) krows.add((long)hh * S + k0 + 32 * w, 32, (long)hh * S + S);
    }
    wg.check();
  }
  krows.expect_once(name + " dK/dV rows");
  check_sweeps(name, swept, roles, [&](int kt) { return (S + BK - 1) / BK - kt * BKV / BK; });
}

// ---------------------------------------------------------------------------
// dK/dV at D = 256 in one pass: attn_dkv_q256_kernel. Grid = heads x 64-key
// blocks; each workgroup sweeps 32-query granules from its block's diagonal on
// (at least 4, an even number). Regions 0-4: the Q slots (Q and lse), 5-7: the
// dO slots (dO and delta), 8-9: the P buffers, 10-11: the dS buffers (by
// granule parity; the two key blocks' halves of a buffer are one region),
// 20 + w: wave w's K / V row staging (waves 0-3, 16 KB each from Q slot 1 on).
// Roles: A (waves 0, 2), B (1, 3), A' (4, 6), B' (5, 7); the light waves A'
// and B' issue the rings' loads.
// ---------------------------------------------------------------------------
static void check_dkv256q(int bh, int Sq, int Sk, bool causal) {
  const int BKV = 64, BG = 32, W = 8, nk = (Sk + BKV - 1) / BKV;
  const int qs = kDkv256qQSlots, ds = kDkv256qDoSlots;
  const std::string name = std::string("dkv_q256") + (causal ? " causal" : "") + " bh" + std::to_string(bh) + " Sq" +
                           std::to_string(Sq) + " Sk" + std::to_string(Sk);
  Coverage cells((long)bh * Sk * 2);
  for (int block = 0; block < bh * nk; ++block) {
    const int head = block % bh, kt = block / bh;
    for (int w = 0; w < W; ++w) {
      const int blk = (w >> 1) & 1, slab = w >= 4 ? 1 : 0;
      for (int r = kt * BKV + 32 * blk; r < std::min(kt * BKV + 32 * blk + 32, Sk); ++r)
        if ((w & 1) == 0) cells.add(((long)head * Sk + r) * 2 + slab, 1, (long)bh * Sk * 2);  // dV (A, A')
    }
  }
  cells.expect_once(name + " dV (row, slab)");
  // Staging of wave w (0-3): bytes [16896 + 16384 w, + 16384), inside Q slots 1-4 (16896 bytes each).
  constexpr long kSlot = 16896;
  auto staging = [&](int w) {
    std::vector<int> r;
    const long lo = kSlot + 16384L * w, hi = lo + 16384;
    for (int i = 0; i < qs; ++i)
      if (kSlot * i < hi && lo < kSlot * (i + 1)) r.push_back(i);
    if (lo + 16384 > kSlot * qs) r.push_back(99);  // past the Q ring: must not happen
    r.push_back(20 + w);
    return r;
  };
  for (int kt = 0; kt < nk; ++kt) {
    const int k0 = kt * BKV;
    const int first = causal ? k0 / BG : 0;
    int nh = std::max((Sq + BG - 1) / BG - first, 4);
    nh += nh & 1;
    if (first * BG > (causal ? k0 : 0) || (first + nh) * BG < Sq) fail(name + ": a sweep misses queries");
    Workgroup wg(W, name + " kt" + std::to_string(kt));
    // Light waves w = 4 .. 7 issue four Q and four dO blocks a granule, plus lse (wave 4) and delta (wave 5).
    auto issue = [&](int x) {
      if (x < nh)
        for (int w = 4; w < W; ++w) wg.issue(w, {x % qs}, 1000 + x, 4 + (w == 4 ? 1 : 0));
    };
    auto issue_do = [&](int x) {
      if (x < nh)
        for (int w = 4; w < W; ++w) wg.issue(w, {5 + x % ds}, 2000 + x, 4 + (w == 5 ? 1 : 0));
    };
    for (int w = 0; w < 4; ++w) wg.issue(w, staging(w), 3000 + w, 16);
    issue(0);
    wg.barrier_all(0);
    for (int w = 0; w < 4; ++w) wg.read(w, 20 + w, 3000 + w);
    wg.barrier_all(-1);
    for (int h = -1; h <= nh + 1; ++h) {
      if (h >= 0) wg.barrier_all(0);
      for (int w = 0; w < W; ++w) {
        const int role = (w & 1) + (w >= 4 ? 2 : 0);  // 0 A, 1 B, 2 A', 3 B'
        if (role == 0) {
          if (h + 1 < nh) wg.read(w, (h + 1) % qs, 1000 + h + 1);      // S of h + 1: Q rows
          if (h >= 0 && h < nh) wg.read(w, h % qs, 1000 + h);         // softmax of h: lse
          if (h >= 1 && h <= nh) wg.read(w, 5 + (h - 1) % ds, 2000 + h - 1);  // dV of h - 1: dO^T
        } else if (role == 1) {
          if (h >= 0 && h < nh) wg.read(w, 5 + h % ds, 2000 + h);     // dP of h: dO rows
          if (h >= 1 && h <= nh) {
            wg.read(w, 5 + (h - 1) % ds, 2000 + h - 1);               // dS of h - 1: delta
            wg.read(w, 8 + ((h - 1) & 1), 5000 + h - 1);              // P of h - 1 from A
            wg.read(w, (h - 1) % qs, 1000 + h - 1);                   // dK of h - 1: Q^T
          }
        } else if (role == 2) {
          if (h >= 1 && h <= nh) {
            wg.read(w, 8 + ((h - 1) & 1), 5000 + h - 1);              // P of h - 1 from A
            wg.read(w, 5 + (h - 1) % ds, 2000 + h - 1);               // dV of h - 1: dO^T
          }
        } else {
          if (h >= 2 && h <= nh + 1) {
            wg.read(w, 10 + ((h - 2) & 1), 6000 + h - 2);             // dS of h - 2 from B
            wg.read(w, (h - 2) % qs, 1000 + h - 2);                   // dK of h - 2: Q^T
          }
        }
      }
      issue(q256q_loaded(h));
      issue_do(do256q_loaded(h));
      // A writes P of h, B writes dS of h - 1 (ds_write, no VMEM count): instant fills in this epoch.
      if (h >= 0 && h < nh)
        for (int w = 0; w < 4; w += 2) wg.issue(w, {8 + (h & 1)}, 5000 + h, 0);
      if (h >= 1 && h <= nh)
        for (int w = 1; w < 4; w += 2) wg.issue(w, {10 + ((h - 1) & 1)}, 6000 + h - 1, 0);
    }
    wg.check();
  }
}

// ---------------------------------------------------------------------------
// Wide head dims: attn_fwd_wide_kernel, attn_dq_wide_kernel (128-row query
// tiles), attn_dkv_wide_kernel (128-row key tiles), each over heads x tiles x
// 128-column slabs. Their LDS staging is synchronous (registers -> LDS between
// two workgroup barriers), so what is checked is the grid: every (row, slab)
// of the output written exactly once.
// ---------------------------------------------------------------------------
static void check_wide(int bh, int S, int D) {
  const int nt = (S + 127) / 128, nc = D / 128;
  for (int kind = 0; kind < 3; ++kind) {
    const bool heavy_last = kind < 2;  // forward and dQ: the last query tiles first
    Coverage cells((long)bh * S * nc);
    for (int block = 0; block < bh * nt * nc; ++block) {
      const WideCoord wc = wide_coord(block, bh, nt, heavy_last);
      if (wc.bh < 0 || wc.bh >= bh || wc.tile < 0 || wc.tile >= nt || wc.slab < 0 || wc.slab >= nc) {
        fail("wide: block " + std::to_string(block) + " maps outside the grid");
        continue;
      }
      for (int r = wc.tile * 128; r < std::min(wc.tile * 128 + 128, S); ++r)
        cells.add(((long)wc.bh * S + r) * nc + wc.slab, 1, (long)bh * S * nc);
    }
    cells.expect_once("wide kind " + std::to_string(kind) + " bh" + std::to_string(bh) + " S" + std::to_string(S) +
                      " D" + std::to_string(D));
  }
}

int main() {
  std::vector<int> lengths;
  for (int s = 64; s <= 4096; s += 64) lengths.push_back(s);
  lengths.push_back(8192);
  const int bhs[] = {1, 3, 8, 64};
  int launches = 0;
  for (int bh : bhs)
    for (int S : lengths) {
      // The forward's launch choices (fwd_launch): D = 128 one 8-wave workgroup per CU; D <= 64 the
      // key-split kernel, zig on a resident grid, the split where it applies.
      check_fwd(FwdCfg{128, 8, 1, false, false}, bh, S);
      check_fwd(FwdCfg{256, 4, 1, false, false}, bh, S);  // D = 256: four waves, two slots
      const int nq64 = (S + 127) / 128;
      const bool zig = resident((long long)nq64 * bh, 2, kCus);
      check_fwd(FwdCfg{64, 8, 2, zig, false}, bh, S);
      if (fwd_split_applies(bh, S, kCus)) check_fwd(FwdCfg{64, 8, 2, true, true}, bh, S);
      // dQ (dq_pp_launch): D = 128 4 waves 2 slots; D = 64 resident: 8 waves, key split, zig; else 4 waves.
      check_dq(DqCfg{128, 4, 2, 1, false, false}, bh, S);
      check_dq(DqCfg{128, 8, 3, 1, false, false}, bh, S);  // the three-slot ring the kernel still supports
      check_dq(DqCfg{256, 4, 2, 1, false, false}, bh, S);  // D = 256: four waves, two slots
      if (resident((long long)((S + 127) / 128) * bh, 2, kCus))
        check_dq(DqCfg{64, 8, 2, 2, true, false}, bh, S);
      else
        check_dq(DqCfg{64, 4, 2, 1, false, false}, bh, S);
      // The split dQ and dK/dV where they apply (with a workspace).
      if (split_applies(bh, S, kCus, kDqSplit)) check_dq(DqCfg{64, 8, 2, 2, true, true}, bh, S), ++launches;
      if (split_applies(bh, S, kCus, kDkvSplit)) check_dkv(64, bh, S, true, true), ++launches;
      // dK/dV (dkv_pp_launch): D = 64 zig on a resident grid; D = 128 the role split.
      check_dkv(64, bh, S, resident((long long)((S + 127) / 128) * bh, 2, kCus));
      check_dkv(128, bh, S, false);
      check_dkv256q(bh, S, S, true);  // D = 256: one pass, four roles
      launches += 10;
    }
  for (int bh : {1, 3, 8})
    for (int S : {1, 100, 128, 200, 1000})
      for (int D : {256, 384, 1024}) check_wide(bh, S, D);
  for (int bh : {1, 3})
    for (int sq : {1, 100, 200, 260})
      for (int sk : {1, 100, 260}) check_dkv256q(bh, sq, sk, false), ++launches;
  // The split at the shapes it was built for, and a cut in each place it can fall.
  for (int bh : {5, 6, 8}) {
    check_fwd(FwdCfg{64, 8, 2, true, true}, bh, 8192);
    check_dq(DqCfg{64, 8, 2, 2, true, true}, bh, 8192);
    check_dkv(64, bh, 8192, true, true);
  }
  if (failures) {
    std::fprintf(stderr, "%d schedule check(s) failed\n", failures);
    return 1;
  }
  // Each planted mistake must be caught.
  const char* planted[] = {"", "K loaded a stage late", "V loaded into a slot in use", "waits too shallow",
                           "dQ tile loaded into a slot in use", "O rows written by both halves of a pair",
                           "dK/dV tile loaded a half-step pair early", "split dQ rows written by both shares",
                           "split dK/dV rows written by both shares", "D = 256 Q granule loaded into a slot in use",
                           "D = 256 dO granule loaded into a slot in use",
                           "D = 128 lse row written a half-step late"};
  constexpr int kPlanted = 11;
  quiet = true;
  for (int m = 1; m <= kPlanted; ++m) {
    g_mutation = m;
    const int before = failures;
    check_fwd(FwdCfg{128, 8, 1, false, false}, 2, 1024);
    check_fwd(FwdCfg{256, 4, 1, false, false}, 2, 1024);
    check_fwd(FwdCfg{64, 8, 2, true, true}, 6, 8192);
    check_dq(DqCfg{64, 4, 2, 1, false, false}, 3, 1024);
    check_dq(DqCfg{256, 4, 2, 1, false, false}, 3, 1024);
    check_dq(DqCfg{64, 8, 2, 2, true, true}, 6, 8192);
    check_dkv(128, 2, 1024, false);
    check_dkv(64, 6, 8192, true, true);
    check_dkv256q(2, 1024, 1024, true);
    if (failures == before) {
      std::fprintf(stderr, "planted mistake %d (%s) not caught\n", m, planted[m]);
      return 1;
    }
    failures = before;
  }
  g_mutation = 0;
  quiet = false;
  std::printf("attention schedules: %d launch configurations replayed, all checks passed; %d planted mistakes caught\n",
              launches, kPlanted);
  return 0;
}
