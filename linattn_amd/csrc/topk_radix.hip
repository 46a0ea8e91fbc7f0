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
constexpr uint32_t RX_SPIN_LIMIT = 1u << 20;  // polls before a wait is given up
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
constexpr int RX_CPT = RX_CAND_CAP / TK_NT;  // candidates per thread
constexpr int RX_CPRE = 4;  // of them read before the row state in the last launch
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
  const TkRow rw = tk_row(a.p, gi);
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
// The last launch reads the first RX_CPRE * TK_NT candidate slots that way
// instead (rows collected by the launch before it, the common case).
__global__ __launch_bounds__(TK_NT) void rx_stage_kernel(RxKP a, int launch, int last, int guess) {
  __shared__ uint32_t hist[RX_BINS];
  __shared__ uint32_t eqc[RX_KPT][TK_NW];  // per slot and wave: threshold keys
  __shared__ uint32_t tkc[RX_KPT][TK_NW];  // per slot and wave: keys taken
  __shared__ uint32_t wtmp[2][TK_NW];
  __shared__ uint32_t s_bin, s_above, s_cnt, s_base, s_take;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const TopkKParams &p = a.p;
  const int64_t c = blockIdx.x, gi = blockIdx.y, NG = p.NG;
  const TkRow rw = tk_row(p, gi);
  const int64_t n_v = rw.n_v;
  // thread t holds bins RX_BINS - 1 - RX_BPT t downwards of a histogram
  auto read_bins = [&](const uint32_t *h, uint32_t (&hv)[RX_BPT]) {
#pragma unroll
    for (int e = 0; e < RX_BPT; ++e) hv[e] = h[RX_BINS - 1 - RX_BPT * tid - e];
  };
  // the prefetch: the likely histogram first, then the chunk's scores (loads
  // complete in order, so the pick below waits for the histogram only)
  uint32_t hpre[RX_BPT];
  if (guess >= 0) read_bins(rx_hist(a, gi, (uint32_t)guess), hpre);
  uint64_t cpre[RX_CPRE];
  if (last) {
    const uint64_t *cd = rx_cand(a, gi);
#pragma unroll
    for (int e = 0; e < RX_CPRE; ++e) cpre[e] = cd[tid + e * TK_NT];
  }
  double vraw[RX_KPT];
  {
    const int64_t x0 = c * RX_CHUNK + tid;
    const double *rp = p.scores + rw.br * p.row_stride;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) vraw[j] = x0 + (int64_t)j * TK_NT < n_v ? rp[x0 + (int64_t)j * TK_NT] : 0.0;
  }
  // the row state as scalars (a copy of the whole struct would live in
  // memory); the row's chunk-0 workgroup writes the next launch's copy
  const RxState *sin = a.state + (launch & 1) * NG + gi;
  RxState *sout = a.state + ((launch + 1) & 1) * NG + gi;
  const bool writer = c == 0 && tid == 0;
  const bool init = a.state_in_kernel && launch == 0;
  const RxState s0 = init ? rx_initial(rw, true) : RxState{};
  uint32_t phase = init ? s0.phase : sin->phase;
  if (phase == RX_DONE) {
    if (writer) sout->phase = RX_DONE;
    return;
  }
  uint64_t prefix = init ? s0.prefix : sin->prefix, mask = init ? s0.mask : sin->mask;
  uint32_t need = init ? s0.need : sin->need, pass = init ? s0.pass : sin->pass;
  uint32_t pend = init ? s0.pend : sin->pend;
  int top = init ? s0.top : sin->top;
  const uint32_t ncand = init ? 0u : sin->ncand;
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
    const uint32_t incl = tk_block_incl_scan(csum, wtmp[0], all);
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
    __syncthreads();
    need -= s_above;
    nmatch = s_cnt;
    prefix |= (uint64_t)s_bin << shift;
    mask |= (uint64_t)dm << shift;
    top = shift - 1;
    pass += 1;
    // the whole bin is taken, or every bit is fixed (the rest are index ties)
    phase = (s_cnt == need || shift == 0) ? RX_COUNT : RX_PASS;
    __syncthreads();  // s_* are read before they are written again
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
  // the chunk's keys above / equal to the final threshold (workgroup totals)
  auto count_chunk = [&](int64_t x, const uint64_t (&u)[RX_KPT], uint32_t &gt_c, uint32_t &eq_c) {
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) {
      const uint64_t um = u[j] & mask;
      gt += valid(x, j) && um > prefix;
      eq += valid(x, j) && um == prefix;
    }
    tk_block_incl_scan(gt, wtmp[0], gt_c);
    tk_block_incl_scan(eq, wtmp[1], eq_c);
  };
  // writes chunk x's selected keys from output position base on, taking its
  // first take_eq threshold keys (index order within the chunk)
  auto write_chunk = [&](int64_t x, const uint64_t (&u)[RX_KPT], uint32_t base, uint32_t take_eq) {
    const int64_t x0 = x * RX_CHUNK + tid;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) {
      const uint64_t b = __ballot(valid(x, j) && (u[j] & mask) == prefix);
      if (lane == 0) eqc[j][w] = (uint32_t)__popcll(b);
    }
    __syncthreads();
    uint32_t take_bits = 0, eq_run = 0;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) {
      const uint64_t um = u[j] & mask;
      const bool is_gt = valid(x, j) && um > prefix;
      const bool is_eq = valid(x, j) && um == prefix;
      const uint64_t b = __ballot(is_eq);
      uint32_t rank = eq_run + (uint32_t)__popcll(b & lt);
#pragma unroll
      for (int y = 0; y < TK_NW; ++y) rank += y < w ? eqc[j][y] : 0u;
#pragma unroll
      for (int y = 0; y < TK_NW; ++y) eq_run += eqc[j][y];
      const bool take = is_gt || (is_eq && rank < take_eq);
      const uint64_t tb = __ballot(take);
      if (lane == 0) tkc[j][w] = (uint32_t)__popcll(tb);
      take_bits |= (uint32_t)take << j;
    }
    __syncthreads();
    uint32_t pos_run = base;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) {
      const bool take = (take_bits >> j) & 1u;
      const uint64_t tb = __ballot(take);
      uint32_t pos = pos_run + (uint32_t)__popcll(tb & lt);
#pragma unroll
      for (int y = 0; y < TK_NW; ++y) pos += y < w ? tkc[j][y] : 0u;
#pragma unroll
      for (int y = 0; y < TK_NW; ++y) pos_run += tkc[j][y];
      if (take) {
        const int64_t i = x0 + (int64_t)j * TK_NT;
        if (ord1) {
          if ((int64_t)pos < p.width) oi[pos] = (int32_t)i;
        } else if (pos < K) {
          a.cand_sc[gi * p.k + pos] = key_to_double(u[j]);
          a.cand_id[gi * p.k + pos] = (int32_t)i;
        }
      }
    }
    __syncthreads();  // eqc / tkc are read before the next chunk writes them
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

  if (phase == RX_PASS && last) {
    // ------------------------------------------- one-workgroup finish --
    if (c != 0) return;
    uint64_t u[RX_KPT];
    while (phase == RX_PASS) {
      for (int b = tid; b < RX_BINS; b += TK_NT) hist[b] = 0u;
      __syncthreads();
      for (int64_t x = 0; x < a.C; ++x) {
        load(x, u);
        hist_chunk(x, u);
      }
      __syncthreads();
      pick(hist);
    }
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
      write_chunk(x, u, base, take_eq);
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
    const uint32_t incl = tk_block_incl_scan(mine, wtmp[0], tot);
    if (tid == 0 && tot)
      s_base = __hip_atomic_fetch_add(rx_ccount(a, gi), tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
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
    uint64_t ck[RX_CPT];
#pragma unroll
    for (int e = 0; e < RX_CPT; ++e) {
      const uint32_t i = (uint32_t)(tid + e * TK_NT);
      ck[e] = e < RX_CPRE && last ? cpre[e] : i < nc ? cd[i] : 0ull;
    }
    phase = RX_PASS;
    while (phase == RX_PASS) {
      for (int b = tid; b < RX_BINS; b += TK_NT) hist[b] = 0u;
      __syncthreads();
      int shift;
      uint32_t dm;
      digit(shift, dm);
#pragma unroll
      for (int e = 0; e < RX_CPT; ++e)
        if ((uint32_t)(tid + e * TK_NT) < nc && (ck[e] & mask) == prefix)
          atomicAdd(&hist[(uint32_t)(ck[e] >> shift) & dm], 1u);
      __syncthreads();
      pick(hist);
    }
  }

  if (phase == RX_PASS) {
    for (int b = tid; b < RX_BINS; b += TK_NT) hist[b] = 0u;
    __syncthreads();
    hist_chunk(c, u);
    __syncthreads();
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
    bool ok = true;
    int64_t hi = c - 1;  // the window's nearest chunk
    while (hi >= 0) {
      const int64_t x = hi - lane;
      uint64_t r = x >= 0 ? __hip_atomic_load(&rec[x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : RX_INC;
      const uint64_t inc = __ballot((r & RX_INC) != 0);
      const uint64_t none = __ballot((r >> 62) == 0);
      // lanes up to and including the nearest inclusive record (all of them
      // when there is none) must have published
      const uint64_t upto = inc ? (inc & (~inc + 1)) * 2 - 1 : ~0ull;
      if (none & upto) {
        if (++spins > RX_SPIN_LIMIT) {
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
        __hip_atomic_fetch_or(&la_dev_status, (uint32_t)LA_DEV_TOPK_TIMEOUT, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
        s_base = 0xffffffffu;
      }
    }
  }
  __syncthreads();
  if (s_base == 0xffffffffu) return;  // the wait was given up: this chunk writes nothing
  write_chunk(c, u, s_base, s_take);
  pad(c * TK_NT + tid, a.C * TK_NT);
  if (writer) sout->phase = RX_DONE;
}

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

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
            align256(p.NG * 8);
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
  base += align256(p.NG * a.row_words * 4);
  base += align256(p.NG * 8);  // the rows' ready words (RadixRowPrep)
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
    const int guess = s == launches - 1 ? -1 : s - (hist0_external ? 0 : 1);
    rx_stage_kernel<<<grid, TK_NT, 0, st>>>(a, s, s == launches - 1 ? 1 : 0, guess);
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
