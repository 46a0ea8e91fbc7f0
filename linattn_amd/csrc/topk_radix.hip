// Row top-k split over many workgroups per row: long rows, few of them (the
// decode indexer of config C5: 131072 keys per sequence, top-4096).
//
// A row is cut into chunks of RX_CHUNK keys; workgroup (c, r) of a launch owns
// chunk c of row r (thread t: keys c * RX_CHUNK + 256 j + t, j < RX_KPT).  The
// selection is an MSB-first radix select over the 64-bit order keys run as a
// fixed sequence of launches of one kernel, rx_stage_kernel, each of which
// advances every row by one stage:
//   stage s < RX_PASSES  histogram one RX_RB-bit digit of the keys that still
//                        match the threshold prefix;
//   RX_COUNT             count each chunk's keys above / equal to the final
//                        threshold;
//   RX_WRITE             write the selected indices in increasing index order
//                        (order 1), or the candidate (score, index) rows that
//                        topk_launch then sorts (order 0).
// Inside a stage a workgroup never waits for another one.  Each adds its
// histogram (or counts) with device-scope atomics and then takes a ticket;
// the workgroup that draws the last ticket of its row finishes the stage for
// the row (picks the threshold bin, or turns the chunk counts into output
// offsets) and writes the row's next stage, which the next launch reads.  The
// last workgroup only waits for atomics the others have already issued (it
// re-reads the sums until every key is counted); it needs no other workgroup
// to be resident or to make progress, so the launches are ordinary ones.
// Rows that finish early do nothing in the remaining launches.
//
// The selection equals tk_select's over the whole row: the K largest keys,
// threshold ties taken lowest index first.
#include <algorithm>

#include "topk.h"
#include "topk_select.h"

namespace la {

constexpr int RX_KPT = 16;                              // keys per thread
constexpr int64_t RX_CHUNK = (int64_t)TK_NT * RX_KPT;  // keys per workgroup
constexpr int RX_RB = 11;                              // radix digit bits
constexpr int RX_BINS = 1 << RX_RB;
constexpr int RX_BPT = RX_BINS / TK_NT;                // bins per thread when picking
constexpr int RX_PASSES = (64 + RX_RB - 1) / RX_RB;
constexpr int RX_COUNT = RX_PASSES, RX_WRITE = RX_PASSES + 1, RX_DONE = RX_PASSES + 2;
constexpr int RX_LAUNCHES = RX_PASSES + 2;             // stage launches after the set-up
constexpr uint32_t RX_SPIN_LIMIT = 1u << 24;           // polls of the last workgroup's wait

// Status bits raised by kernels of this library on the current device, read
// and cleared by la_device_status.
__device__ uint32_t la_dev_status;

// Per-row state.  The set-up kernel initialises it; during a launch only the
// row's last workgroup writes it (after every other one has read it).
struct RxRow {
  uint64_t prefix, mask;  // threshold bits fixed so far
  uint32_t need;          // keys equal to the prefix still to take (lowest index first)
  uint32_t expect;        // keys of the row that match the prefix
  uint32_t stage;         // the stage the next launch runs for this row
  int32_t top;            // highest bit of the next digit
  uint32_t err;           // a wait of the last workgroup ran out (not expected)
  uint32_t pad0;
  uint32_t ticket[RX_LAUNCHES];
  uint32_t counted[RX_PASSES];  // keys added into each pass's histogram so far
  uint32_t pad[64 - 10 - RX_LAUNCHES - RX_PASSES];
};
static_assert(sizeof(RxRow) == 256, "RxRow layout");

struct RxKP {
  TopkKParams p;
  RxRow *rows;        // [NG]
  uint32_t *hist;     // [NG][RX_PASSES][RX_BINS]
  uint32_t *chunk;    // [NG][C][4]: gt + 1, eq + 1 (published), offset, eq keys taken
  double *cand_sc;    // order 0: candidate rows [NG][k], sorted afterwards
  int32_t *cand_id;
  int64_t C;
};

__device__ __forceinline__ uint32_t rx_load(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void rx_add(uint32_t *p, uint32_t x) {
  __hip_atomic_fetch_add(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Zeroes a row's histograms and chunk records and sets its first stage: the
// radix passes, or straight to counting when every valid key is taken.  One
// workgroup per row.
__global__ __launch_bounds__(TK_NT) void rx_setup_kernel(RxKP a) {
  const int64_t gi = blockIdx.x;
  const TkRow rw = tk_row(a.p, gi);
  uint4 *h = (uint4 *)(a.hist + gi * RX_PASSES * RX_BINS);
  for (int i = threadIdx.x; i < RX_PASSES * RX_BINS / 4; i += TK_NT) h[i] = make_uint4(0, 0, 0, 0);
  uint4 *ch = (uint4 *)(a.chunk + gi * a.C * 4);
  for (int64_t i = threadIdx.x; i < a.C; i += TK_NT) ch[i] = make_uint4(0, 0, 0, 0);
  uint32_t *r = (uint32_t *)(a.rows + gi);
  if (threadIdx.x < 64) r[threadIdx.x] = 0u;
  __syncthreads();
  if (threadIdx.x == 0) {
    RxRow *st = a.rows + gi;
    const uint32_t K = (uint32_t)rw.K, n_v = (uint32_t)rw.n_v;
    st->need = K >= n_v ? n_v : K;  // all keys taken: every key matches the empty prefix
    st->expect = n_v;
    st->stage = K >= n_v ? (uint32_t)RX_COUNT : 0u;
    st->top = 63;
  }
}

__global__ __launch_bounds__(TK_NT) void rx_stage_kernel(RxKP a) {
  __shared__ uint32_t hist[RX_BINS];
  __shared__ uint32_t eqc[RX_KPT][TK_NW];  // per slot and wave: threshold keys
  __shared__ uint32_t tkc[RX_KPT][TK_NW];  // per slot and wave: keys taken
  __shared__ uint32_t wtmp[2][TK_NW];
  __shared__ uint32_t s_last, s_bin, s_above, s_cnt, s_err;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const TopkKParams &p = a.p;
  const int64_t c = blockIdx.x, gi = blockIdx.y;
  RxRow *st = a.rows + gi;
  const uint32_t stage = st->stage;
  if (stage >= (uint32_t)RX_DONE || (int64_t)c >= a.C) return;
  const TkRow rw = tk_row(p, gi);
  const int64_t n_v = rw.n_v;
  const uint64_t prefix = st->prefix, mask = st->mask;
  const uint32_t need = st->need, expect = st->expect;
  const int64_t c0 = c * RX_CHUNK + tid;
  auto valid = [&](int j) { return c0 + (int64_t)j * TK_NT < n_v; };
  uint64_t u[RX_KPT];
  {
    const double *rp = p.scores + rw.br * p.row_stride;
    double v[RX_KPT];
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) v[j] = valid(j) ? rp[c0 + (int64_t)j * TK_NT] : 0.0;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) u[j] = ord_key(v[j]);
  }
  uint32_t *chunk = a.chunk + (gi * a.C + c) * 4;

  // ---------------------------------------------------------------- pass --
  if (stage < (uint32_t)RX_COUNT) {
    const int top = st->top;
    const int shift = top >= RX_RB - 1 ? top - (RX_RB - 1) : 0;
    const uint32_t dm = (2u << (top - shift)) - 1u;
    for (int b = tid; b < RX_BINS; b += TK_NT) hist[b] = 0u;
    __syncthreads();
    uint32_t mine = 0;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) {
      if (valid(j) && (u[j] & mask) == prefix) {
        atomicAdd(&hist[(uint32_t)(u[j] >> shift) & dm], 1u);
        ++mine;
      }
    }
    __syncthreads();
    uint32_t *gh = a.hist + (gi * RX_PASSES + stage) * RX_BINS;
    for (int b = tid; b < RX_BINS; b += TK_NT) {
      const uint32_t x = hist[b];
      if (x) rx_add(&gh[b], x);
    }
    uint32_t tot;
    tk_block_incl_scan(mine, wtmp[1], tot);
    if (tid == 0) {
      if (tot) rx_add(&st->counted[stage], tot);
      const uint32_t t = __hip_atomic_fetch_add(&st->ticket[stage], 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      s_last = t == (uint32_t)(a.C - 1);
      s_err = 0;
    }
    __syncthreads();
    if (!s_last) return;
    // The last workgroup: every other one has issued its atomics.  Wait until
    // the row's count shows every matching key, then read the histogram until
    // its bins sum to the same number (bins only grow, so that read saw every
    // bin's final count).  Thread t holds bins RX_BINS - 1 - RX_BPT t downwards.
    if (tid == 0) {
      uint32_t spins = 0;
      while (rx_load(&st->counted[stage]) < expect && ++spins < RX_SPIN_LIMIT)
        __builtin_amdgcn_s_sleep(1);
      s_err = spins >= RX_SPIN_LIMIT;
    }
    __syncthreads();
    uint32_t h[RX_BPT], csum = 0, incl = 0, all = 0;
    for (uint32_t spins = 0; !s_err; ++spins) {
      csum = 0;
#pragma unroll
      for (int e = 0; e < RX_BPT; ++e) {
        h[e] = rx_load(&gh[RX_BINS - 1 - RX_BPT * tid - e]);
        csum += h[e];
      }
      incl = tk_block_incl_scan(csum, wtmp[0], all);
      if (all == expect) break;
      if (spins >= RX_SPIN_LIMIT) {
        if (tid == 0) s_err = 1;
        __syncthreads();
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (s_err) {
      if (tid == 0) {
        st->err = 1u;
        st->stage = (uint32_t)RX_WRITE;  // the write stage reports the row as failed
      }
      return;
    }
    // the bin holding the need-th largest matching key
    if (incl >= need && incl - csum < need) {
      uint32_t acc = incl - csum;
      bool found = false;
#pragma unroll
      for (int e = 0; e < RX_BPT; ++e) {
        if (!found && acc + h[e] >= need) {
          s_bin = (uint32_t)(RX_BINS - 1 - RX_BPT * tid - e);
          s_above = acc;
          s_cnt = h[e];
          found = true;
        }
        acc += h[e];
      }
    }
    __syncthreads();
    if (tid == 0) {
      const uint32_t nd = need - s_above;
      st->prefix = prefix | ((uint64_t)s_bin << shift);
      st->mask = mask | ((uint64_t)dm << shift);
      st->need = nd;
      st->expect = s_cnt;
      st->top = shift - 1;
      // the whole bin is taken, or every bit is fixed (the rest are index ties)
      st->stage = (s_cnt == nd || shift == 0) ? (uint32_t)RX_COUNT : stage + 1u;
    }
    return;
  }

  // --------------------------------------------------------------- count --
  if (stage == (uint32_t)RX_COUNT) {
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) {
      const uint64_t um = u[j] & mask;
      gt += valid(j) && um > prefix;
      eq += valid(j) && um == prefix;
    }
    uint32_t gt_c, eq_c;
    tk_block_incl_scan(gt, wtmp[0], gt_c);
    tk_block_incl_scan(eq, wtmp[1], eq_c);
    if (tid == 0) {
      // published as count + 1, so that 0 reads as "not yet written"
      __hip_atomic_store(&chunk[0], gt_c + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&chunk[1], eq_c + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t t = __hip_atomic_fetch_add(&st->ticket[RX_COUNT], 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      s_last = t == (uint32_t)(a.C - 1);
    }
    __syncthreads();
    if (!s_last) return;
    // The last workgroup turns the chunk counts into output offsets: chunk x
    // writes after the keys the chunks before it select and takes the first
    // need - (threshold keys before it) of its own threshold keys.
    uint32_t gt_run = 0, eq_run = 0, bad = 0;
    for (int64_t x0 = 0; x0 < a.C; x0 += TK_NT) {
      const int64_t x = x0 + tid;
      uint32_t g1 = 0, e1 = 0;
      if (x < a.C) {
        uint32_t *cx = a.chunk + (gi * a.C + x) * 4;
        uint32_t spins = 0;
        g1 = rx_load(&cx[0]);
        e1 = rx_load(&cx[1]);
        while ((g1 == 0 || e1 == 0) && ++spins < RX_SPIN_LIMIT) {
          __builtin_amdgcn_s_sleep(1);
          g1 = rx_load(&cx[0]);
          e1 = rx_load(&cx[1]);
        }
        if (g1 == 0 || e1 == 0) bad = 1;
      }
      const uint32_t gx = g1 ? g1 - 1u : 0u, ex = e1 ? e1 - 1u : 0u;
      uint32_t gtot, etot;
      const uint32_t gi_incl = tk_block_incl_scan(gx, wtmp[0], gtot);
      const uint32_t ei_incl = tk_block_incl_scan(ex, wtmp[1], etot);
      if (x < a.C) {
        const uint32_t gb = gt_run + gi_incl - gx, eb = eq_run + ei_incl - ex;
        uint32_t *cx = a.chunk + (gi * a.C + x) * 4;
        cx[2] = gb + min(need, eb);
        cx[3] = eb >= need ? 0u : min(need - eb, ex);
      }
      gt_run += gtot;
      eq_run += etot;
    }
    uint32_t nbad;
    tk_block_incl_scan(bad, wtmp[0], nbad);
    if (tid == 0) {
      if (nbad) st->err = 1u;
      st->stage = (uint32_t)RX_WRITE;
    }
    return;
  }

  // --------------------------------------------------------------- write --
  const bool ord1 = p.order == 1;
  const uint32_t K = (uint32_t)rw.K;
  int32_t *oi = p.out_idx + rw.orow * p.width;
  const int64_t stride = a.C * TK_NT;
  if (st->err) {  // a wait ran out: the row comes back empty (-1) and is reported
    if (ord1) {
      for (int64_t x = c * TK_NT + tid; x < p.width; x += stride) oi[x] = -1;
      if (c == 0 && tid == 0 && p.out_count) p.out_count[rw.orow] = -1;
    } else {
      for (int64_t x = c * TK_NT + tid; x < p.k; x += stride) {
        a.cand_sc[gi * p.k + x] = __longlong_as_double((long long)0xffffffffffffffffull);
        a.cand_id[gi * p.k + x] = -1;
      }
    }
    if (c == 0 && tid == 0)
      __hip_atomic_fetch_or(&la_dev_status, (uint32_t)LA_DEV_TOPK_TIMEOUT, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
  } else {
    const uint32_t base = chunk[2], take_eq = chunk[3];
    const uint64_t lt = lanemask_lt(lane);
    // ranks of the threshold keys in index order (slot-major within the chunk)
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) {
      const uint64_t b = __ballot(valid(j) && (u[j] & mask) == prefix);
      if (lane == 0) eqc[j][w] = (uint32_t)__popcll(b);
    }
    __syncthreads();
    uint32_t take_bits = 0, eq_run = 0;
#pragma unroll
    for (int j = 0; j < RX_KPT; ++j) {
      const uint64_t um = u[j] & mask;
      const bool is_gt = valid(j) && um > prefix;
      const bool is_eq = valid(j) && um == prefix;
      const uint64_t b = __ballot(is_eq);
      uint32_t rank = eq_run + (uint32_t)__popcll(b & lt);
#pragma unroll
      for (int x = 0; x < TK_NW; ++x) rank += x < w ? eqc[j][x] : 0u;
#pragma unroll
      for (int x = 0; x < TK_NW; ++x) eq_run += eqc[j][x];
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
      for (int x = 0; x < TK_NW; ++x) pos += x < w ? tkc[j][x] : 0u;
#pragma unroll
      for (int x = 0; x < TK_NW; ++x) pos_run += tkc[j][x];
      if (take) {
        const int64_t i = c0 + (int64_t)j * TK_NT;
        if (ord1) {
          if ((int64_t)pos < p.width) oi[pos] = (int32_t)i;
        } else if (pos < K) {
          a.cand_sc[gi * p.k + pos] = key_to_double(u[j]);
          a.cand_id[gi * p.k + pos] = (int32_t)i;
        }
      }
    }
    // padding after the K winners, and the count
    if (ord1) {
      for (int64_t x = K + c * TK_NT + tid; x < p.width; x += stride) oi[x] = -1;
      if (c == 0 && tid == 0 && p.out_count) p.out_count[rw.orow] = (int32_t)min((int64_t)K, p.width);
    } else {
      // the lowest key (all-ones pattern) and index -1: sorted after every real one
      for (int64_t x = K + c * TK_NT + tid; x < p.k; x += stride) {
        a.cand_sc[gi * p.k + x] = __longlong_as_double((long long)0xffffffffffffffffull);
        a.cand_id[gi * p.k + x] = -1;
      }
    }
  }
  if (tid == 0) {
    const uint32_t t = __hip_atomic_fetch_add(&st->ticket[RX_WRITE], 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    if (t == (uint32_t)(a.C - 1)) st->stage = (uint32_t)RX_DONE;
  }
}

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

RadixPlan radix_plan(const TopkKParams &p) {
  RadixPlan R;
  if (p.n >= ((int64_t)1 << 31)) return R;
  R.C = ceil_div(p.n, RX_CHUNK);
  R.bytes = align256(p.NG * (int64_t)sizeof(RxRow)) + align256(p.NG * RX_PASSES * RX_BINS * 4) +
            align256(p.NG * R.C * 16);
  if (p.order == 0) R.bytes += align256(p.NG * p.k * 8) + align256(p.NG * p.k * 4);
  return R;
}

int topk_radix_launch(const TopkKParams &p, const RadixPlan &R, void *ws, hipStream_t st) {
  if ((uintptr_t)ws % 16 != 0) return fail(LA_ERR_INVALID, "topk: workspace not 16-byte aligned");
  LA_REQUIRE(p.NG < 65536, "topk: at most 65535 long rows per call");
  char *base = (char *)ws;
  RxKP a{};
  a.p = p;
  a.C = R.C;
  a.rows = (RxRow *)base;
  base += align256(p.NG * (int64_t)sizeof(RxRow));
  a.hist = (uint32_t *)base;
  base += align256(p.NG * RX_PASSES * RX_BINS * 4);
  a.chunk = (uint32_t *)base;
  base += align256(p.NG * R.C * 16);
  if (p.order == 0) {
    a.cand_sc = (double *)base;
    a.cand_id = (int32_t *)(base + align256(p.NG * p.k * 8));
  }
  rx_setup_kernel<<<dim3((unsigned)p.NG), TK_NT, 0, st>>>(a);
  LA_LAUNCHED();
  const dim3 grid((unsigned)R.C, (unsigned)p.NG);
  for (int s = 0; s < RX_LAUNCHES; ++s) {
    rx_stage_kernel<<<grid, TK_NT, 0, st>>>(a);
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
