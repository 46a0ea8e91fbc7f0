// Row top-k split over many workgroups per row: long rows, few of them (the
// decode indexer of config C5: 131072 keys per sequence, top-4096).
//
// A row is cut into chunks of RX_CHUNK keys; workgroup (c, r) of a launch owns
// chunk c of row r (thread t: keys c * RX_CHUNK + 256 j + t, j < RX_KPT).  The
// selection is an MSB-first radix select over the 64-bit order keys, run as a
// fixed sequence of launches of one kernel, rx_stage_kernel; every launch
// moves each row one phase on:
//   PASS    histogram one RX_RB-bit digit of the keys that match the
//           threshold prefix (device-scope atomics into the row's histogram
//           of that pass);
//   COUNT   count each chunk's keys above / equal to the final threshold;
//   WRITE   write the selected indices in increasing index order (order 1),
//           or the candidate (score, index) rows that topk_launch then sorts
//           (order 0).
// A launch begins by picking the threshold bin of the pass the previous
// launch histogrammed: every workgroup of the row reads the complete
// histogram (the launch boundary orders it) and makes the same pick, so no
// workgroup ever waits for another and no launch needs the others resident.
// The row state a launch reads is the one the previous launch wrote (two
// copies, by launch parity), written by the row's chunk-0 workgroup.  Rows
// that finish early do nothing in the remaining launches.
//
// The sequence is short: RX_FAST_PASSES chunk-parallel passes (three, 28
// bits fixed, settle the threshold of scores spread over their leading bits;
// the fourth runs only for rows they leave open), the count, and a last
// launch that writes.  A row still undecided by
// then (keys tied over most of their bits) is finished in that last launch
// by one workgroup, which loops over the row's chunks.
//
// The first pass's histogram (the top RX_RB bits) may come from the kernel
// that writes the scores (the decode indexer, indexer_decode16_kernel),
// which saves a launch and a read of the scores.
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
enum { RX_PASS = 0, RX_COUNT = 1, RX_WRITE = 2, RX_DONE = 3 };
// digit passes run chunk-parallel: up to four (39 bits fixed); rows that
// need more finish in one workgroup in the last launch.  A row whose
// threshold the first three settle (28 bits: scores spread over their
// leading bits) counts and writes a launch early and skips the rest.
constexpr int RX_FAST_PASSES = 4;
// digit histograms in the workspace per row: the chunk-parallel passes and
// the one the last launch picks from (the finishing workgroup keeps its own
// in LDS)
constexpr int RX_HISTS = RX_FAST_PASSES + 1;
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
  uint32_t phase;         // RX_PASS, RX_COUNT, RX_WRITE or RX_DONE
  int32_t top;            // highest bit of pass `pass`'s digit
  uint32_t pad[3];
};
static_assert(sizeof(RxState) == 48, "RxState layout");

struct RxKP {
  TopkKParams p;
  RxState *state;     // [2][NG]
  uint32_t *hist;     // [NG][RX_HISTS][RX_BINS]
  uint32_t *chunk;    // [NG][C][2]: keys above / equal to the final threshold
  double *cand_sc;    // order 0: candidate rows [NG][k], sorted afterwards
  int32_t *cand_id;
  int64_t C;
};

// Zeroes a row's histograms and sets its first phase: the radix passes
// (pass 0 pending a pick when the scores' kernel histograms it), or straight
// to counting when every valid key is taken.  One workgroup per row.
__global__ __launch_bounds__(TK_NT) void rx_setup_kernel(RxKP a, int hist0_external) {
  const int64_t gi = blockIdx.x;
  const TkRow rw = tk_row(a.p, gi);
  uint4 *h = (uint4 *)(a.hist + gi * RX_HISTS * RX_BINS);
  for (int i = threadIdx.x; i < RX_HISTS * RX_BINS / 4; i += TK_NT) h[i] = make_uint4(0, 0, 0, 0);
  if (threadIdx.x == 0) {
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
    a.state[gi] = s;
  }
}

// Launch `launch` of a row's stage sequence.  Launches before the last one
// run the phases chunk-parallel (above).  The last launch writes the rows
// that have reached the write phase the same way; a row that has not (its
// threshold still undecided after the chunk-parallel passes: keys tied over
// many of their leading bits) is finished by its chunk-0 workgroup alone,
// which runs the remaining passes, then counts and writes chunk after chunk
// in index order (one read of the row per pass, one for the count and the
// write together), while the row's other workgroups exit.
// `guess`: the pass whose histogram this launch picks from in the common case
// (-1: none); it is read before the row state, together with the chunk's
// scores, so that the launch waits for one memory round trip instead of three.
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
  if (guess >= 0) read_bins(a.hist + (gi * RX_HISTS + guess) * RX_BINS, hpre);
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
  uint32_t phase = sin->phase;
  if (phase == RX_DONE) {
    if (writer) sout->phase = RX_DONE;
    return;
  }
  uint64_t prefix = sin->prefix, mask = sin->mask;
  uint32_t need = sin->need, pass = sin->pass, pend = sin->pend;
  int top = sin->top;
  auto publish = [&](uint32_t next_phase, uint32_t next_pend) {
    sout->prefix = prefix;
    sout->mask = mask;
    sout->need = need;
    sout->pass = pass;
    sout->pend = next_pend;
    sout->phase = next_phase;
    sout->top = top;
  };
  const uint32_t K = (uint32_t)rw.K;
  const bool ord1 = p.order == 1;
  int32_t *oi = p.out_idx + rw.orow * p.width;
  const uint64_t lt = lanemask_lt(lane);
  uint32_t *chunk = a.chunk + gi * a.C * 2;

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

  if (last && !(phase == RX_WRITE && !pend)) {
    // ------------------------------------------- one-workgroup finish --
    if (c != 0) return;
    if (pend) pick(a.hist + (gi * RX_HISTS + pass) * RX_BINS);
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

  // the pick of the pass the previous launch histogrammed: every workgroup
  // of the row reads the complete histogram and makes the same pick
  if (pend) {
    if ((int)pass == guess)
      pick_bins(hpre);
    else
      pick(a.hist + (gi * RX_HISTS + pass) * RX_BINS);
  }
  uint64_t u[RX_KPT];
#pragma unroll
  for (int j = 0; j < RX_KPT; ++j) u[j] = ord_key(vraw[j]);

  if (phase == RX_PASS) {
    for (int b = tid; b < RX_BINS; b += TK_NT) hist[b] = 0u;
    __syncthreads();
    hist_chunk(c, u);
    __syncthreads();
    uint32_t *gh = a.hist + (gi * RX_HISTS + pass) * RX_BINS;
    for (int b = tid; b < RX_BINS; b += TK_NT) {
      const uint32_t x = hist[b];
      if (x) __hip_atomic_fetch_add(&gh[b], x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (writer) publish(RX_PASS, 1u);
    return;
  }

  if (phase == RX_COUNT) {
    uint32_t gt_c, eq_c;
    count_chunk(c, u, gt_c, eq_c);
    if (tid == 0) {
      chunk[2 * c] = gt_c;
      chunk[2 * c + 1] = eq_c;
    }
    if (writer) publish(RX_WRITE, 0u);
    return;
  }

  // ---------------------------------------------------------------- write --
  // this chunk's output offset and the threshold keys it takes, from the
  // counts of the chunks before it
  {
    uint32_t gb = 0, eb = 0;
    for (int64_t x = tid; x < c; x += TK_NT) {
      gb += chunk[2 * x];
      eb += chunk[2 * x + 1];
    }
    uint32_t gtot, etot;
    tk_block_incl_scan(gb, wtmp[0], gtot);
    tk_block_incl_scan(eb, wtmp[1], etot);
    if (tid == 0) {
      const uint32_t ex = chunk[2 * c + 1];
      s_base = gtot + min(need, etot);
      s_take = etot >= need ? 0u : min(need - etot, ex);
    }
    __syncthreads();
  }
  write_chunk(c, u, s_base, s_take);
  pad(c * TK_NT + tid, a.C * TK_NT);
  if (writer) sout->phase = RX_DONE;
}

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

RadixPlan radix_plan(const TopkKParams &p) {
  RadixPlan R;
  if (p.n >= ((int64_t)1 << 31)) return R;
  R.C = ceil_div(p.n, RX_CHUNK);
  R.bytes = align256(2 * p.NG * (int64_t)sizeof(RxState)) +
            align256(p.NG * RX_HISTS * RX_BINS * 4) + align256(p.NG * R.C * 8);
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
  a.hist = (uint32_t *)base;
  base += align256(p.NG * RX_HISTS * RX_BINS * 4);
  a.chunk = (uint32_t *)base;
  base += align256(p.NG * R.C * 8);
  if (p.order == 0) {
    a.cand_sc = (double *)base;
    a.cand_id = (int32_t *)(base + align256(p.NG * p.k * 8));
  }
  return a;
}

uint32_t *radix_hist0(const TopkKParams &p, void *ws) {
  return (uint32_t *)((char *)ws + align256(2 * p.NG * (int64_t)sizeof(RxState)));
}
int64_t radix_hist_stride() { return (int64_t)RX_HISTS * RX_BINS; }

int topk_radix_setup(const TopkKParams &p, const RadixPlan &R, void *ws, bool hist0_external,
                     hipStream_t st) {
  if ((uintptr_t)ws % 16 != 0) return fail(LA_ERR_INVALID, "topk: workspace not 16-byte aligned");
  LA_REQUIRE(p.NG < 65536, "topk: at most 65535 long rows per call");
  rx_setup_kernel<<<dim3((unsigned)p.NG), TK_NT, 0, st>>>(rx_args(p, R, ws), hist0_external ? 1 : 0);
  LA_LAUNCHED();
  return LA_OK;
}

int topk_radix_finish(const TopkKParams &p, const RadixPlan &R, void *ws, bool hist0_external,
                      hipStream_t st) {
  const RxKP a = rx_args(p, R, ws);
  const dim3 grid((unsigned)R.C, (unsigned)p.NG);
  // chunk-parallel launches for the passes that settle the threshold of
  // scores spread over their leading bits (the first pass may come from the
  // scores' kernel) and the count; the last launch writes (or finishes a
  // row whose threshold is still open in one workgroup)
  const int launches = RX_FAST_PASSES - (hist0_external ? 1 : 0) + 2;
  for (int s = 0; s < launches; ++s) {
    // launch s picks pass s (pass 0 histogrammed by the scores' kernel) or
    // s - 1 in the common case; the last launch only writes
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
  return topk_radix_finish(p, R, ws, false, st);
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
  const int rc = prefill_status(&more, clear != 0, st);
  if (rc != LA_OK) return rc;
  *bits |= more;
  return LA_OK;
}
