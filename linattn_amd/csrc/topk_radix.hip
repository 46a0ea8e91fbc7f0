// Row top-k split over many workgroups per row: long rows, few of them (the
// decode indexer of config C5: 131072 keys per sequence, top-4096).
//
// A row is cut into chunks of RX_CHUNK keys; workgroup (c, r) of a launch owns
// chunk c of row r (thread t: keys c * RX_CHUNK + 256 j + t, j < RX_KPT).  The
// selection is an MSB-first radix select over the 64-bit order keys, run as a
// fixed sequence of launches of one kernel, rx_stage_kernel; every launch
// moves each row one phase on:
//   PASS    histogram one digit of the keys that match the threshold prefix
//           (device-scope atomics into the row's histogram of that pass);
//   CAND    (when at most RX_CAND_CAP keys match the prefix) collect those
//           keys into the row's candidate list instead;
//   COUNT   count each chunk's keys above / equal to the final threshold and
//           write the chunk's selected indices in increasing index order
//           (order 1), or the candidate (score, index) rows that topk_launch
//           then sorts (order 0), after the counts of the chunks before it.
// A launch begins by picking the threshold bin of the pass the previous
// launch histogrammed: every workgroup of the row reads the complete
// histogram (the launch boundary orders it) and makes the same pick; a row
// whose keys were collected is settled instead by every workgroup from the
// candidate list alone (the remaining digits, histogrammed in LDS), and
// counts and writes in the same launch.  The row state a launch reads is the
// one the previous launch wrote (two copies, by launch parity), written by
// the row's chunk-0 workgroup.  Rows that finish early do nothing in the
// remaining launches.
//
// The output offset of a chunk is the number of keys the chunks before it
// select: each chunk publishes its counts in one 64-bit record, then its
// inclusive prefix, and looks back over the records of the chunks before it
// (decoupled look-back).  Workgroup (c, r) waits only for workgroups (x, r),
// x < c, of lower linear id; those are dispatched before it and publish
// before they wait themselves, so no wait depends on a workgroup that is not
// yet running, and no launch needs its workgroups resident together.  The
// waits are bounded (a hardware-fault guard: past the bound the chunk's
// output is skipped and LA_DEV_TOPK_TIMEOUT raised).
//
// The sequence is short: RX_FAST_PASSES chunk-parallel passes at most (28
// bits: digits of 11, 6 and 11 bits), then one launch more.  Scores spread
// over their leading bits leave a few hundred keys in the threshold bin
// after two digits: they are collected, and the last launch settles, counts
// and writes.  A row still undecided after the last chunk-parallel pass and
// never collected (over RX_CAND_CAP keys tied over 28 bits) is finished in
// the last launch by one workgroup, which loops over the row's chunks.
//
// The first pass's histogram (the top RX_RB bits) may come from the kernel
// that writes the scores (the decode indexer, indexer_decode16_kernel),
// which saves a launch and a read of the scores; that kernel may also clear
// the rows' records and the first launch start from the initial state, which
// saves the set-up launch.  C5 then runs the indexer and three launches.
//
// The selection equals tk_select's over the whole row: the K largest keys,
// threshold ties taken lowest index first.
#include <algorithm>
#include <atomic>
#include <cstddef>

#include "topk.h"
#include "topk_select.h"

namespace la {

constexpr int RX_KPT = 16;                              // keys per thread
constexpr int64_t RX_CHUNK = (int64_t)TK_NT * RX_KPT;  // keys per workgroup
constexpr int RX_BPT = RX_BINS / TK_NT;                // bins per thread when picking
enum { RX_PASS = 0, RX_COUNT = 1, RX_CAND = 2, RX_DONE = 3 };
// Chunk records (64 bits): the flag in bits 62-63 (0 none, RX_AGG the chunk's
// own counts, RX_INC the counts of chunks 0..c), keys above the threshold in
// bits 31-61, keys equal to it in bits 0-30 (a row holds < 2^31 keys).
constexpr uint64_t RX_AGG = 1ull << 62, RX_INC = 2ull << 62;
constexpr uint32_t RX_SPIN_LIMIT = 1u << 20;  // polls before a wait is given up (default)
// digit passes run chunk-parallel: up to three (28 bits fixed); a row that
// needs more, and whose keys matching the threshold prefix were not few
// enough to be collected (RX_CAND_CAP), finishes in one workgroup in the
// last launch.
constexpr int RX_FAST_PASSES = 3;
// When at most this many keys of a row match the threshold prefix after a
// pick, the row's workgroups collect them (the keys only) instead of
// histogramming the next digit, and in the next launch every workgroup of the
// row settles the threshold from them alone, in LDS, then counts and writes:
// the remaining passes cost no launches.  (About 450 keys of a C5 row match
// after the first two digits.)
constexpr int RX_CAND_CAP = 4096;
constexpr int RX_CPT = RX_CAND_CAP / TK_NT;  // candidates per thread (workgroup settle)
// Up to RX_WCAP candidates (the common case) every wave settles alone, with
// 8-bit digits and a 256-bin histogram of its own: no workgroup barrier.
constexpr int RX_WCAP = 1024;
constexpr int RX_WCPL = RX_WCAP / 64;  // candidates per lane (wave settle)
constexpr int RX_CPRE = 8;             // of them read before the row state in the last launch
// digit histograms in the workspace per row, one per chunk-parallel pass (the
// finishing workgroup keeps its own in LDS)
constexpr int RX_HISTS = RX_FAST_PASSES;
// Bits of pass i's digit: RX_RB, except 6 for the second pass.  The first
// digit (sign and the top of the exponent) leaves a whole binade range of
// scores in its threshold bin (about 29 000 of the 131 072 keys of a C5 row),
// which the second pass histograms; at 6 bits each chunk adds at most 64
// bins into the row's histogram with device atomics instead of ~600 at 11
// bits.  Three passes fix 28 bits, four 39.
__device__ __forceinline__ int rx_digit_bits(uint32_t pass) { return pass == 1 ? 6 : RX_RB; }

// Status bits raised by kernels of this library on the current device, read
// and cleared by la_device_status.
__device__ uint32_t la_dev_status;
__device__ __forceinline__ void raise_timeout() {
  __hip_atomic_fetch_or(&la_dev_status, (uint32_t)LA_DEV_TOPK_TIMEOUT, __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT);
}

// Per-row state between launches.
struct RxState {
  uint64_t prefix, mask;  // threshold bits fixed so far
  uint32_t need;          // keys equal to the prefix still to take (lowest index first)
  uint32_t pass;          // the pass histogrammed next (or last, while pend)
  uint32_t pend;          // pass `pass`'s histogram is complete and not yet picked
  uint32_t phase;         // RX_PASS, RX_COUNT or RX_DONE
  int32_t top;            // highest bit of pass `pass`'s digit
  uint32_t ncand;         // RX_CAND: keys collected (those matching the prefix)
  uint32_t pad[2];
};
static_assert(sizeof(RxState) == 48, "RxState layout");

struct RxKP {
  TopkKParams p;
  RxState *state;     // [2][NG]
  // per row, row_words 32-bit words: the digit histograms [RX_HISTS][RX_BINS],
  // the chunk records (uint64_t [C]), the candidates' count (4 words) and the
  // candidate keys (uint64_t [RX_CAND_CAP])
  uint32_t *rows;
  int64_t row_words;
  double *cand_sc;    // order 0: candidate rows [NG][k], sorted afterwards
  int32_t *cand_id;
  int64_t C;
  int32_t state_in_kernel;  // launch 0 starts from the initial state (no set-up launch)
  int32_t row32;            // tk_row's quotients fit 32-bit arithmetic
  uint64_t *epoch;          // the scores kernel's ready-word epoch (RadixRowPrep)
  uint32_t spin_limit;      // polls before a cross-workgroup wait is given up
};

__device__ __forceinline__ uint32_t *rx_hist(const RxKP &a, int64_t gi, uint32_t pass) {
  return a.rows + gi * a.row_words + (int64_t)pass * RX_BINS;
}
__device__ __forceinline__ uint64_t *rx_rec(const RxKP &a, int64_t gi) {
  return (uint64_t *)(a.rows + gi * a.row_words + RX_HISTS * RX_BINS);
}
__device__ __forceinline__ uint32_t *rx_ccount(const RxKP &a, int64_t gi) {
  return a.rows + gi * a.row_words + RX_HISTS * RX_BINS + 2 * a.C;
}
__device__ __forceinline__ uint64_t *rx_cand(const RxKP &a, int64_t gi) {
  return (uint64_t *)(a.rows + gi * a.row_words + RX_HISTS * RX_BINS + 2 * a.C + 4);
}

// The state a row starts from: the radix passes (pass 0 pending a pick when
// the scores' kernel histograms it), or straight to counting when every
// valid key is taken.
__device__ __forceinline__ RxState rx_initial(const TkRow &rw, bool hist0_external) {
  const uint32_t K = (uint32_t)rw.K, n_v = (uint32_t)rw.n_v;
  RxState s{};
  s.top = 63;
  s.need = K;
  if (K == 0 || K >= n_v) {  // none or every valid key taken: the empty prefix decides
    s.phase = RX_COUNT;
  } else {
    s.phase = RX_PASS;
    s.pend = hist0_external ? 1u : 0u;
  }
  return s;
}

// Zeroes a row's histograms and chunk records and sets its first phase.  One
// workgroup per row.
__global__ __launch_bounds__(TK_NT) void rx_setup_kernel(RxKP a, int hist0_external) {
  const int64_t gi = blockIdx.x;
  const TkRow rw = a.row32 ? tk_row<true>(a.p, gi) : tk_row<false>(a.p, gi);
  uint4 *h = (uint4 *)(a.rows + gi * a.row_words);
  for (int64_t i = threadIdx.x; i < a.row_words / 4; i += TK_NT) h[i] = make_uint4(0, 0, 0, 0);
  if (threadIdx.x == 0) a.state[gi] = rx_initial(rw, hist0_external != 0);
}

// Launch `launch` of a row's stage sequence, chunk-parallel (above).  In the
// last launch, a row whose threshold is still undecided after the
// chunk-parallel passes (keys tied over many of their leading bits) is
// finished by its chunk-0 workgroup alone, which runs the remaining passes,
// then counts and writes chunk after chunk in index order (one read of the
// row per pass, one for the count and the write together), while the row's
// other workgroups exit.
// `guess`: the pass whose histogram this launch picks from in the common case
// (-1: none); it is read before the row state, together with the chunk's
// scores, so that the launch waits for one memory round trip instead of three.
// The last launch reads the first RX_CPRE * 64 candidate slots that way
// instead (rows collected by the launch before it, the common case).
// R32: the row arithmetic in 32 bits (RxKP::row32).  LAST: the last launch
// of the sequence.  Every prefetch load is issued unconditionally (clamped
// addresses), so that the compiler can wait for the early ones alone.
template <bool R32, bool LAST>
__global__ __launch_bounds__(TK_NT) void rx_stage_kernel(RxKP a, int launch, int guess) {
  constexpr bool last = LAST;
  __shared__ uint32_t hist[RX_BINS];
  __shared__ __align__(16) uint32_t whist[TK_NW][256];  // per wave (wave settle)
  __shared__ uint32_t eqc[RX_KPT][TK_NW];  // per slot and wave: threshold keys
  __shared__ uint32_t tkc[RX_KPT][TK_NW];  // per slot and wave: keys taken
  __shared__ uint32_t wtmp[2][TK_NW];
  __shared__ uint32_t s_bin, s_above, s_cnt, s_base, s_take;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const TopkKParams &p = a.p;
  const int64_t c = blockIdx.x, gi = blockIdx.y, NG = p.NG;
  // the row state, read first and whole (48 bytes in three 16-byte words, so
  // that the loads are issued together and their round trip overlaps the
  // row's index arithmetic); the row's chunk-0 workgroup writes the next
  // launch's copy
  const RxState *sin = a.state + (launch & 1) * NG + gi;
  RxState *sout = a.state + ((launch + 1) & 1) * NG + gi;
  const bool init = a.state_in_kernel && launch == 0;
  // the scores kernel's ready-word epoch moves on (it read it before this
  // launch began), so the next call waits for a value of its own
  if (init && c == 0 && gi == 0 && tid == 0) *a.epoch += 1;
  // (read in the first launch too, where the initial state replaces it:
  // no branch keeps the loads apart from their use)
  uint4 sv[3];
  {
    const uint4 *sp = (const uint4 *)sin;
#pragma unroll
    for (int i = 0; i < 3; ++i) sv[i] = sp[i];
  }
  static_assert(offsetof(RxState, prefix) == 0 && offsetof(RxState, mask) == 8 &&
                    offsetof(RxState, need) == 16 && offsetof(RxState, pass) == 20 &&
                    offsetof(RxState, pend) == 24 && offsetof(RxState, phase) == 28 &&
                    offsetof(RxState, top) == 32 && offsetof(RxState, ncand) == 36,
                "RxState words");
  const TkRow rw = tk_row<R32>(p, gi);
  const int64_t n_v = rw.n_v;
  // thread t holds bins RX_BINS - 1 - RX_BPT t downwards of a histogram
  auto read_bins = [&](const uint32_t *h, uint32_t (&hv)[RX_BPT]) {
#pragma unroll
    for (int e = 0; e < RX_BPT; ++e) hv[e] = h[RX_BINS - 1 - RX_BPT * tid - e];
  };
  // the state as scalars (a copy of the whole struct would live in memory)
  const bool writer = c == 0 && tid == 0;
  const RxState s0 = init ? rx_initial(rw, true) : RxState{};
  uint32_t phase = init ? s0.phase : sv[1].w;
  uint64_t prefix = init ? s0.prefix : ((uint64_t)sv[0].y << 32 | sv[0].x);
  uint64_t mask = init ? s0.mask : ((uint64_t)sv[0].w << 32 | sv[0].z);
  uint32_t need = init ? s0.need : sv[1].x, pass = init ? s0.pass : sv[1].y;
  uint32_t pend = init ? s0.pend : sv[1].z;
  int top = init ? s0.top : (int)sv[2].x;
  const uint32_t ncand = init ? 0u : sv[2].y;
  // the prefetch: the likely histogram, then the candidates, then the
  // chunk's scores (the pick waits for the histogram only, the settle for
  // the candidates)
  uint32_t hpre[RX_BPT];
  if (!LAST) read_bins(rx_hist(a, gi, (uint32_t)max(guess, 0)), hpre);
  uint64_t cpre[RX_CPRE];
  if (LAST) {
    const uint64_t *cd = rx_cand(a, gi);
#pragma unroll
    for (int e = 0; e < RX_CPRE; ++e) cpre[e] = cd[lane + e * 64];  // (every wave: the same)
  }
  __builtin_amdgcn_sched_barrier(0);  // (issued before the scores)
  double vraw[RX_KPT];
  {
    // (keys past the valid prefix read key 0 of the row, then count as invalid)
    const int64_t x0 = c * RX_CHUNK + tid;
    const double *rp = p.scores + rw.br * p.row_stride;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) {
      const int64_t i = x0 + (int64_t)j * TK_NT;
      vraw[j] = rp[i < n_v ? i : 0];
    }
  }
  if (phase == RX_DONE) {
    if (writer) sout->phase = RX_DONE;
    return;
  }
  auto publish = [&](uint32_t next_phase, uint32_t next_pend, uint32_t next_ncand) {
    sout->prefix = prefix;
    sout->mask = mask;
    sout->need = need;
    sout->pass = pass;
    sout->pend = next_pend;
    sout->phase = next_phase;
    sout->top = top;
    sout->ncand = next_ncand;
  };
  // the keys matching the prefix: all valid keys before any pick, the
  // picked bin's count after one (unknown otherwise)
  uint32_t nmatch = mask == 0 ? (uint32_t)n_v : 0xffffffffu;
  const uint32_t K = (uint32_t)rw.K;
  const bool ord1 = p.order == 1;
  int32_t *oi = p.out_idx + rw.orow * p.width;
  const uint64_t lt = lanemask_lt(lane);
  uint64_t *rec = rx_rec(a, gi);

  // the order keys of chunk x (thread t: keys x * RX_CHUNK + t + 256 j)
  auto load = [&](int64_t x, uint64_t (&u)[RX_KPT]) {
    const int64_t x0 = x * RX_CHUNK + tid;
    const double *rp = p.scores + rw.br * p.row_stride;
    double v[RX_KPT];
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) v[j] = x0 + (int64_t)j * TK_NT < n_v ? rp[x0 + (int64_t)j * TK_NT] : 0.0;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) u[j] = ord_key(v[j]);
  };
  auto valid = [&](int64_t x, int j) { return x * RX_CHUNK + tid + (int64_t)j * TK_NT < n_v; };
  // the digit below the fixed bits (the width of pass `pass`): its shift
  // and mask
  auto digit = [&](int &shift, uint32_t &dm) {
    const int wd = rx_digit_bits(pass);
    shift = top >= wd - 1 ? top - (wd - 1) : 0;
    dm = (2u << (top - shift)) - 1u;
  };
  // picks the bin of the need-th largest matching key from the bins hv of a
  // complete histogram of the current digit (read_bins) and moves the state
  // past it
  auto pick_bins = [&](const uint32_t (&hv)[RX_BPT]) {
    int shift;
    uint32_t dm;
    digit(shift, dm);
    uint32_t csum = 0, all;
#pragma unroll
    for (int e = 0; e < RX_BPT; ++e) csum += hv[e];
    if (tid == 0) s_cnt = 0;  // a found bin holds at least one key
    const uint32_t incl = tk_block_incl_scan<TK_NT, true>(csum, wtmp[0], all);
    if (incl >= need && incl - csum < need) {
      uint32_t acc = incl - csum;
      bool found = false;
#pragma unroll
      for (int e = 0; e < RX_BPT; ++e) {
        if (!found && acc + hv[e] >= need) {
          s_bin = (uint32_t)(RX_BINS - 1 - RX_BPT * tid - e);
          s_above = acc;
          s_cnt = hv[e];
          found = true;
        }
        acc += hv[e];
      }
    }
    lds_barrier();
    need -= s_above;
    nmatch = s_cnt;
    prefix |= (uint64_t)s_bin << shift;
    mask |= (uint64_t)dm << shift;
    top = shift - 1;
    pass += 1;
    // the whole bin is taken, or every bit is fixed (the rest are index ties)
    phase = (s_cnt == need || shift == 0) ? RX_COUNT : RX_PASS;
    if (s_cnt == 0) {  // a histogram short of need keys: counts were left out
      phase = RX_DONE;
      if (tid == 0) raise_timeout();
    }
    lds_barrier();  // s_* are read before they are written again
  };
  auto pick = [&](const uint32_t *h) {
    uint32_t hv[RX_BPT];
    read_bins(h, hv);
    pick_bins(hv);
  };
  // adds the chunk's keys that match the prefix to the LDS histogram
  auto hist_chunk = [&](int64_t x, const uint64_t (&u)[RX_KPT]) {
    int shift;
    uint32_t dm;
    digit(shift, dm);
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j)
      if (valid(x, j) && (u[j] & mask) == prefix) atomicAdd(&hist[(uint32_t)(u[j] >> shift) & dm], 1u);
  };
  // the chunk's keys above / equal to the final threshold (workgroup totals:
  // one reduction of both counts, each below 2^16, packed in a word)
  auto count_chunk = [&](int64_t x, const uint64_t (&u)[RX_KPT], uint32_t &gt_c, uint32_t &eq_c) {
    uint32_t v = 0;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) {
      const uint64_t um = u[j] & mask;
      v += valid(x, j) ? (um > prefix ? 0x10000u : um == prefix ? 1u : 0u) : 0u;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o, 64);
    if (lane == 0) wtmp[0][w] = v;
    lds_barrier();
    uint32_t t = 0;
#pragma unroll
    for (int y = 0; y < TK_NW; ++y) t += wtmp[0][y];
    lds_barrier();  // wtmp is read before it is written again
    gt_c = t >> 16;
    eq_c = t & 0xffffu;
  };
  // the exclusive prefix of per-(slot, wave) counts cnt[j][y] in key order
  // (slot-major): lane l of every wave reads entry l (RX_KPT x TK_NW = 64)
  // after the barrier, the wave scans them, and entry (j, w) is then read
  // from lane 4 j + w
  static_assert(RX_KPT * TK_NW == 64, "one count per lane");
  const int wu = __builtin_amdgcn_readfirstlane(w);  // (w as a uniform value)
  // stores the wave's per-slot counts (uniform) into cnt[j][w]: lane j writes
  // slot j's
  auto put_counts = [&](uint32_t (&cnt)[RX_KPT][TK_NW], const uint32_t (&v)[RX_KPT]) {
    uint32_t mine = 0;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) mine = lane == j ? v[j] : mine;
    if (lane < RX_KPT) cnt[lane][w] = mine;
  };
  auto slot_scan = [&](const uint32_t (&cnt)[RX_KPT][TK_NW]) {
    const uint32_t v = (&cnt[0][0])[lane];
    uint32_t incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t y = (uint32_t)__shfl_up((int)incl, off, 64);
      if (lane >= off) incl += y;
    }
    return incl - v;
  };
  // writes chunk x's selected keys from output position base on, taking its
  // first take_eq of its eq_c threshold keys (index order within the chunk);
  // more: another chunk follows (the LDS counts are reused)
  auto write_chunk = [&](int64_t x, const uint64_t (&u)[RX_KPT], uint32_t base, uint32_t take_eq,
                         uint32_t eq_c, bool more) {
    const int64_t x0 = x * RX_CHUNK + tid;
    uint32_t take_bits = 0;
    if (take_eq == 0 || take_eq >= eq_c) {  // all or none of the threshold keys
#pragma unroll
      for (int j = 0; j < RX_KPT; ++j) {
        const uint64_t um = u[j] & mask;
        const bool take = valid(x, j) && (um > prefix || (um == prefix && take_eq != 0));
        take_bits |= (uint32_t)take << j;
      }
    } else {  // the first take_eq threshold keys in index order
      uint32_t ce[RX_KPT];
#pragma unroll
      for (int j = 0; j < RX_KPT; ++j) ce[j] = (uint32_t)__popcll(__ballot(valid(x, j) && (u[j] & mask) == prefix));
      put_counts(eqc, ce);
      lds_barrier();
      const uint32_t ex = slot_scan(eqc);
#pragma unroll
      for (int j = 0; j < RX_KPT; ++j) {
        const uint64_t um = u[j] & mask;
        const bool is_eq = valid(x, j) && um == prefix;
        const uint64_t b = __ballot(is_eq);
        const uint32_t rank =
            (uint32_t)__builtin_amdgcn_readlane((int)ex, j * TK_NW + wu) + (uint32_t)__popcll(b & lt);
        const bool take = (valid(x, j) && um > prefix) || (is_eq && rank < take_eq);
        take_bits |= (uint32_t)take << j;
      }
    }
    uint32_t ct[RX_KPT];
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) ct[j] = (uint32_t)__popcll(__ballot((take_bits >> j) & 1u));
    put_counts(tkc, ct);
    lds_barrier();
    const uint32_t ex = slot_scan(tkc);
    // position of slot j's key among the chunk's taken keys, from base on
    auto slot_pos = [&](int j) {
      const uint64_t tb = __ballot((take_bits >> j) & 1u);
      return base + (uint32_t)__builtin_amdgcn_readlane((int)ex, j * TK_NW + wu) + (uint32_t)__popcll(tb & lt);
    };
    const int32_t i0 = (int32_t)x0;  // (a row holds < 2^31 keys)
    if (ord1) {
      const uint32_t wmax = (uint32_t)min(p.width, (int64_t)0xffffffff);
#pragma unroll
      for (int j = 0; j < RX_KPT; ++j) {
        const uint32_t pos = slot_pos(j);
        if (((take_bits >> j) & 1u) && pos < wmax) oi[pos] = i0 + j * TK_NT;
      }
    } else {
      double *csc = a.cand_sc + gi * p.k;
      int32_t *cid = a.cand_id + gi * p.k;
#pragma unroll
      for (int j = 0; j < RX_KPT; ++j) {
        const uint32_t pos = slot_pos(j);
        if (((take_bits >> j) & 1u) && pos < K) {
          csc[pos] = key_to_double(u[j]);
          cid[pos] = i0 + j * TK_NT;
        }
      }
    }
    if (more) lds_barrier();  // eqc / tkc are read before the next chunk writes them
  };
  // padding after the K winners (positions first + stride * m), and the count
  auto pad = [&](int64_t first, int64_t stride) {
    if (ord1) {
      for (int64_t y = K + first; y < p.width; y += stride) oi[y] = -1;
      if (writer && p.out_count) p.out_count[rw.orow] = (int32_t)min((int64_t)K, p.width);
    } else {
      // a double whose order key is 0 (below every real score) and index -1
      for (int64_t y = K + first; y < p.k; y += stride) {
        a.cand_sc[gi * p.k + y] = __longlong_as_double((long long)0xffffffffffffffffull);
        a.cand_id[gi * p.k + y] = -1;
      }
    }
  };

  // the pick of the pass the previous launch histogrammed: every workgroup
  // of the row reads the complete histogram and makes the same pick
  if (pend) {
    if ((int)pass == guess)
      pick_bins(hpre);
    else
      pick(rx_hist(a, gi, pass));
  }
  // a row whose histogram came out short (a wait given up): nothing more
  auto give_up = [&]() {
    if (writer) sout->phase = RX_DONE;
  };
  if (phase == RX_DONE) return give_up();

  if (phase == RX_PASS && last) {
    // ------------------------------------------- one-workgroup finish --
    if (c != 0) return;
    uint64_t u[RX_KPT];
    while (phase == RX_PASS) {
      for (int b = tid; b < RX_BINS; b += TK_NT) hist[b] = 0u;
      lds_barrier();
      for (int64_t x = 0; x < a.C; ++x) {
        load(x, u);
        hist_chunk(x, u);
      }
      lds_barrier();
      pick(hist);
    }
    if (phase == RX_DONE) return give_up();
    // count and write together, chunk after chunk in index order: chunk x
    // writes after the keys the chunks before it select and takes the
    // first need - (threshold keys before it) of its own threshold keys
    uint32_t gt_before = 0, eq_before = 0;
    for (int64_t x = 0; x < a.C; ++x) {
      load(x, u);
      uint32_t gt_c, eq_c;
      count_chunk(x, u, gt_c, eq_c);
      const uint32_t base = gt_before + min(need, eq_before);
      const uint32_t take_eq = eq_before >= need ? 0u : min(need - eq_before, eq_c);
      write_chunk(x, u, base, take_eq, eq_c, true);
      gt_before += gt_c;
      eq_before += eq_c;
    }
    pad(tid, TK_NT);
    if (writer) sout->phase = RX_DONE;
    return;
  }

  uint64_t u[RX_KPT];
#pragma unroll
  for (int j = 0; j < RX_KPT; ++j) u[j] = ord_key(vraw[j]);

  if (phase == RX_PASS && nmatch <= (uint32_t)RX_CAND_CAP) {
    // ------------------------------------------------ collect candidates --
    // the chunk's keys that match the prefix, appended to the row's
    // candidates (in any order: the next launch needs the multiset only)
    uint32_t mine = 0, tot;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) mine += valid(c, j) && (u[j] & mask) == prefix;
    const uint32_t incl = tk_block_incl_scan<TK_NT, true>(mine, wtmp[0], tot);
    if (tid == 0 && tot)
      s_base = __hip_atomic_fetch_add(rx_ccount(a, gi), tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds_barrier();
    if (tot) {
      uint64_t *cd = rx_cand(a, gi);
      uint32_t pos = s_base + incl - mine;
#pragma unroll
      for (int j = 0; j < RX_KPT; ++j)
        if (valid(c, j) && (u[j] & mask) == prefix) {
          if (pos < (uint32_t)RX_CAND_CAP) cd[pos] = u[j];  // (the bin's count bounds pos)
          ++pos;
        }
    }
    if (writer) publish(RX_CAND, 0u, nmatch);
    return;
  }

  if (phase == RX_CAND) {
    // ------------------------------------------- settle from candidates --
    // the remaining digits over the collected keys, each workgroup of the
    // row on its own (the same keys, the same picks), then the count and the
    // write below
    const uint32_t nc = min(ncand, (uint32_t)RX_CAND_CAP);
    const uint64_t *cd = rx_cand(a, gi);
    phase = RX_PASS;
    // every wave alone: lane l holds candidates l + 64 e (ck: an array of
    // uint64_t, e below its length); 8-bit digits, bins counted in the wave's
    // own LDS histogram (a wave's LDS operations complete in order), picked
    // with a wave scan
    auto wave_settle = [&](const auto &ck) {
      constexpr int NPL = (int)(sizeof(ck) / sizeof(ck[0]));
      uint32_t *wh = whist[w];
      while (phase == RX_PASS) {
        const int shift = top >= 7 ? top - 7 : 0;
        const uint32_t dm = (2u << (top - shift)) - 1u;
        *(uint4 *)&wh[4 * lane] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int e = 0; e < NPL; ++e)
          if ((uint32_t)(lane + 64 * e) < nc && (ck[e] & mask) == prefix)
            atomicAdd(&wh[(uint32_t)(ck[e] >> shift) & dm], 1u);
        // lane l: bins 255 - 4 l downwards (.w the highest of its four)
        const uint4 hv = *(const uint4 *)&wh[252 - 4 * lane];
        const uint32_t cs = hv.x + hv.y + hv.z + hv.w;
        uint32_t incl = cs;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const uint32_t y = (uint32_t)__shfl_up((int)incl, off, 64);
          if (lane >= off) incl += y;
        }
        const uint64_t hit = __ballot(incl >= need && incl - cs < need);
        if (hit == 0) {  // a candidate list short of need keys: counts were left out
          phase = RX_DONE;
          if (lane == 0) raise_timeout();
          break;
        }
        const int L = __builtin_ctzll(hit);
        uint32_t acc = (uint32_t)__builtin_amdgcn_readlane((int)(incl - cs), L);
        const uint32_t h3 = (uint32_t)__builtin_amdgcn_readlane((int)hv.w, L);
        const uint32_t h2 = (uint32_t)__builtin_amdgcn_readlane((int)hv.z, L);
        const uint32_t h1 = (uint32_t)__builtin_amdgcn_readlane((int)hv.y, L);
        const uint32_t h0 = (uint32_t)__builtin_amdgcn_readlane((int)hv.x, L);
        uint32_t bin, cnt;
        if (acc + h3 >= need) {
          bin = 255 - 4 * L, cnt = h3;
        } else if (acc += h3, acc + h2 >= need) {
          bin = 254 - 4 * L, cnt = h2;
        } else if (acc += h2, acc + h1 >= need) {
          bin = 253 - 4 * L, cnt = h1;
        } else {
          acc += h1;
          bin = 252 - 4 * L, cnt = h0;
        }
        need -= acc;
        prefix |= (uint64_t)bin << shift;
        mask |= (uint64_t)dm << shift;
        top = shift - 1;
        phase = (cnt == need || shift == 0) ? RX_COUNT : RX_PASS;
      }
    };
    if (LAST && nc <= (uint32_t)(RX_CPRE * 64)) {
      wave_settle(cpre);  // the prefetched slots hold them all
    } else if (nc <= (uint32_t)RX_WCAP) {
      uint64_t ck[RX_WCPL];
#pragma unroll
      for (int e = 0; e < RX_WCPL; ++e) {
        const uint32_t i = (uint32_t)(lane + 64 * e);
        ck[e] = i < nc ? cd[i] : 0ull;
      }
      wave_settle(ck);
    } else {
      // the whole workgroup: thread t holds candidates t + 256 e
      uint64_t ck[RX_CPT];
#pragma unroll
      for (int e = 0; e < RX_CPT; ++e) {
        const uint32_t i = (uint32_t)(tid + e * TK_NT);
        ck[e] = i < nc ? cd[i] : 0ull;
      }
      while (phase == RX_PASS) {
        for (int b = tid; b < RX_BINS; b += TK_NT) hist[b] = 0u;
        lds_barrier();
        int shift;
        uint32_t dm;
        digit(shift, dm);
#pragma unroll
        for (int e = 0; e < RX_CPT; ++e)
          if ((uint32_t)(tid + e * TK_NT) < nc && (ck[e] & mask) == prefix)
            atomicAdd(&hist[(uint32_t)(ck[e] >> shift) & dm], 1u);
        lds_barrier();
        pick(hist);
      }
    }
    if (phase == RX_DONE) return give_up();
  }

  if (phase == RX_PASS) {
    for (int b = tid; b < RX_BINS; b += TK_NT) hist[b] = 0u;
    lds_barrier();
    hist_chunk(c, u);
    lds_barrier();
    uint32_t *gh = rx_hist(a, gi, pass);
    for (int b = tid; b < RX_BINS; b += TK_NT) {
      const uint32_t x = hist[b];
      if (x) __hip_atomic_fetch_add(&gh[b], x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (writer) publish(RX_PASS, 1u, 0u);
    return;
  }

  // ------------------------------------------------------ count and write --
  // The chunk's counts, then its output offset and the threshold keys it
  // takes from the counts of the chunks before it (decoupled look-back by
  // wave 0: lanes read the records of chunks c - 1 - lane of a 64-record
  // window, nearest first; a window is summed up to its nearest inclusive
  // record, or whole when it holds only aggregates, then the next window).
  uint32_t gt_c, eq_c;
  count_chunk(c, u, gt_c, eq_c);
  if (w == 0) {
    const uint64_t own = ((uint64_t)gt_c << 31) | (uint64_t)eq_c;
    // (the records carry their data in the word itself: relaxed device-scope
    // atomics suffice, and no fence writes back or drops the caches)
    if (lane == 0 && c > 0) __hip_atomic_store(&rec[c], RX_AGG | own, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t gb = 0, eb = 0, spins = 0;
    bool ok = a.spin_limit > 0 || c == 0;  // (a limit of 0 gives every wait up at once)
    int64_t hi = c - 1;  // the window's nearest chunk
    while (ok && hi >= 0) {
      const int64_t x = hi - lane;
      uint64_t r = x >= 0 ? __hip_atomic_load(&rec[x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : RX_INC;
      const uint64_t inc = __ballot((r & RX_INC) != 0);
      const uint64_t none = __ballot((r >> 62) == 0);
      // lanes up to and including the nearest inclusive record (all of them
      // when there is none) must have published
      const uint64_t upto = inc ? (inc & (~inc + 1)) * 2 - 1 : ~0ull;
      if (none & upto) {
        if (++spins > a.spin_limit) {
          ok = false;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
        continue;
      }
      const bool mine = ((upto >> lane) & 1) != 0;
      uint32_t g = mine ? (uint32_t)((r >> 31) & 0x7fffffffu) : 0u;
      uint32_t e = mine ? (uint32_t)(r & 0x7fffffffu) : 0u;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        g += (uint32_t)__shfl_xor((int)g, o, 64);
        e += (uint32_t)__shfl_xor((int)e, o, 64);
      }
      gb += g;
      eb += e;
      if (inc) break;
      hi -= 64;
    }
    if (lane == 0) {
      if (ok) {
        __hip_atomic_store(&rec[c], RX_INC | (((uint64_t)(gb + gt_c)) << 31) | (uint64_t)(eb + eq_c),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_base = gb + min(need, eb);
        s_take = eb >= need ? 0u : min(need - eb, eq_c);
      } else {
        raise_timeout();
        s_base = 0xffffffffu;
      }
    }
  }
  lds_barrier();
  if (s_base == 0xffffffffu) return;  // the wait was given up: this chunk writes nothing
  write_chunk(c, u, s_base, s_take, eq_c, false);
  pad(c * TK_NT + tid, a.C * TK_NT);
  if (writer) sout->phase = RX_DONE;
}

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// Polls after which a cross-workgroup wait gives up (la_test_set_spin_limit).
static std::atomic<uint32_t> g_spin_limit{RX_SPIN_LIMIT};
uint32_t rx_spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }

// 32-bit words per row: the digit histograms, then the chunk records (a
// multiple of 4 words, so rows stay 16-byte aligned)
static int64_t rx_row_words(int64_t C) {
  return (RX_HISTS * RX_BINS + 2 * C + 4 + 2 * RX_CAND_CAP + 3) / 4 * 4;
}

RadixPlan radix_plan(const TopkKParams &p) {
  RadixPlan R;
  if (p.n >= ((int64_t)1 << 31)) return R;
  R.C = ceil_div(p.n, RX_CHUNK);
  R.bytes = align256(2 * p.NG * (int64_t)sizeof(RxState)) + align256(p.NG * rx_row_words(R.C) * 4) +
            align256((p.NG + 1) * 8);
  if (p.order == 0) R.bytes += align256(p.NG * p.k * 8) + align256(p.NG * p.k * 4);
  return R;
}

static RxKP rx_args(const TopkKParams &p, const RadixPlan &R, void *ws) {
  char *base = (char *)ws;
  RxKP a{};
  a.p = p;
  a.C = R.C;
  a.state = (RxState *)base;
  base += align256(2 * p.NG * (int64_t)sizeof(RxState));
  a.rows = (uint32_t *)base;
  a.row_words = rx_row_words(R.C);
  a.row32 = tk_row_fits_32(p) ? 1 : 0;
  a.spin_limit = rx_spin_limit();
  base += align256(p.NG * a.row_words * 4);
  a.epoch = (uint64_t *)base + p.NG;
  base += align256((p.NG + 1) * 8);  // the rows' ready words and the epoch (RadixRowPrep)
  if (p.order == 0) {
    a.cand_sc = (double *)base;
    a.cand_id = (int32_t *)(base + align256(p.NG * p.k * 8));
  }
  return a;
}

RadixRowPrep radix_row_prep(const TopkKParams &p, const RadixPlan &R, void *ws) {
  const RxKP a = rx_args(p, R, ws);
  RadixRowPrep r;
  r.rows = a.rows;
  r.row_words = a.row_words;
  r.ready = (uint64_t *)((char *)a.rows + align256(p.NG * a.row_words * 4));
  r.epoch = a.epoch;
  return r;
}

int topk_radix_setup(const TopkKParams &p, const RadixPlan &R, void *ws, bool hist0_external,
                     hipStream_t st) {
  if ((uintptr_t)ws % 16 != 0) return fail(LA_ERR_INVALID, "topk: workspace not 16-byte aligned");
  LA_REQUIRE(p.NG < 65536, "topk: at most 65535 long rows per call");
  rx_setup_kernel<<<dim3((unsigned)p.NG), TK_NT, 0, st>>>(rx_args(p, R, ws), hist0_external ? 1 : 0);
  LA_LAUNCHED();
  return LA_OK;
}

int topk_radix_finish(const TopkKParams &p, const RadixPlan &R, void *ws, bool hist0_external,
                      bool state_in_kernel, hipStream_t st) {
  if ((uintptr_t)ws % 16 != 0) return fail(LA_ERR_INVALID, "topk: workspace not 16-byte aligned");
  LA_REQUIRE(p.NG < 65536, "topk: at most 65535 long rows per call");
  LA_REQUIRE(!state_in_kernel || hist0_external,
             "topk: the rows start in the first launch only after an external first pass");
  RxKP a = rx_args(p, R, ws);
  a.state_in_kernel = state_in_kernel ? 1 : 0;
  const dim3 grid((unsigned)R.C, (unsigned)p.NG);
  // one launch per chunk-parallel pass (the first may come from the scores'
  // kernel); a row counts and writes in the launch whose pick settles it, and
  // the last launch finishes a row still open in one workgroup
  const int launches = RX_FAST_PASSES + (hist0_external ? 0 : 1);
  for (int s = 0; s < launches; ++s) {
    // launch s picks pass s (pass 0 histogrammed by the scores' kernel) or
    // s - 1; the last one mostly settles collected rows (no histogram read)
    const bool lst = s == launches - 1;
    const int guess = lst ? -1 : s - (hist0_external ? 0 : 1);
    if (a.row32 && lst)
      rx_stage_kernel<true, true><<<grid, TK_NT, 0, st>>>(a, s, guess);
    else if (a.row32)
      rx_stage_kernel<true, false><<<grid, TK_NT, 0, st>>>(a, s, guess);
    else if (lst)
      rx_stage_kernel<false, true><<<grid, TK_NT, 0, st>>>(a, s, guess);
    else
      rx_stage_kernel<false, false><<<grid, TK_NT, 0, st>>>(a, s, guess);
    LA_LAUNCHED();
  }
  if (p.order == 0) {
    // sorted output: order the K winners of each row by (score desc, index asc)
    TopkKParams f = p;
    f.scores = a.cand_sc;
    f.row_stride = p.k;
    f.n = p.k;
    f.pos_unit = 0;
    f.n_valid_tab = nullptr;
    f.cand_idx = a.cand_id;
    const int rc = topk_launch(f, st);
    if (rc != LA_OK) return rc;
  }
  return LA_OK;
}

int topk_radix_launch(const TopkKParams &p, const RadixPlan &R, void *ws, hipStream_t st) {
  const int rc = topk_radix_setup(p, R, ws, false, st);
  if (rc != LA_OK) return rc;
  return topk_radix_finish(p, R, ws, false, false, st);
}

}  // namespace la

using namespace la;

// The status word read (and, with clear, reset) in one atomic exchange on the
// caller's stream, after the work queued on it: a bit raised by a kernel of
// another stream is either in this read or kept for the next one.
__device__ uint32_t la_dev_status_snap;
__global__ void dev_status_kernel(int clear) {
  la_dev_status_snap = clear ? __hip_atomic_exchange(&la_dev_status, 0u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT)
                             : __hip_atomic_load(&la_dev_status, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
}

extern "C" int la_test_set_spin_limit(uint32_t polls) {
  g_spin_limit.store(polls, std::memory_order_relaxed);
  return LA_OK;
}

extern "C" int la_device_status(uint32_t *bits, int32_t clear, void *stream) {
  LA_REQUIRE(bits != nullptr, "la_device_status: null pointer");
  hipStream_t st = (hipStream_t)stream;
  dev_status_kernel<<<1, 1, 0, st>>>(clear ? 1 : 0);
  LA_LAUNCHED();
  LA_HIP(hipMemcpyFromSymbolAsync(bits, HIP_SYMBOL(la_dev_status_snap), sizeof(uint32_t), 0,
                                  hipMemcpyDeviceToHost, st));
  LA_HIP(hipStreamSynchronize(st));
  // status words of the other source files (each holds its own device symbol)
  uint32_t more = 0;
  int rc = prefill_status(&more, clear != 0, st);
  if (rc != LA_OK) return rc;
  *bits |= more;
  more = 0;
  rc = indexer_status(&more, clear != 0, st);
  if (rc != LA_OK) return rc;
  *bits |= more;
  return LA_OK;
}
