// Row top-k split over many workgroups: long rows, few of them.
//
// A row is cut into chunks of TW_CHUNK keys; workgroup (c, r) holds chunk c
// of row r in registers (TW_KPT order keys per thread, unit
// c * TW_CHUNK + j * 256 + t).  The radix select of tk_select then runs over
// the whole row at once.  Each pass histograms one digit (TW_RB bits) of the
// keys still matching the threshold prefix in LDS, adds the non-empty bins
// into the row's histogram for that pass in global memory (device-scope
// atomics) plus its key count into the row's running count, and waits for
// that count to reach the number of keys the pass counts (known from the
// previous pass); it then reads the histogram back until its bins sum to
// that number too, that is until every chunk's counts are in, and every
// workgroup picks the same threshold bin.  No barrier or fence is needed.
// The passes stop when the threshold bin is taken whole or every bit is
// fixed.  Each chunk then publishes its counts of keys above and equal to
// the threshold and waits only for the chunks before it, whose counts give
// its output offset, so the K winners come out in increasing index order
// with threshold ties taken lowest index first: the selection tk_select
// makes over the whole row.
//
// The waits need every workgroup of a row resident at once: the kernel is
// launched cooperatively (the runtime refuses a grid that cannot be), rows
// go in batches that fit, and every wait is bounded.  A wait that runs out
// marks its row; once every batch (and the final sort) has run,
// tw_finish_kernel pads each marked row with -1, sets its count to -1 and
// raises LA_DEV_TOPK_TIMEOUT in the device status word (la_device_status).
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "topk.h"
#include "topk_select.h"

namespace la {

constexpr int TW_KPT = 16;                             // keys per thread
constexpr int64_t TW_CHUNK = (int64_t)TK_NT * TW_KPT;  // keys per workgroup
constexpr int TW_RB = 11;                              // radix digit bits
constexpr int TW_BINS = 1 << TW_RB;
constexpr int TW_BPT = TW_BINS / TK_NT;               // bins per thread in the scan
constexpr int TW_PASSES = (64 + TW_RB - 1) / TW_RB;
constexpr uint32_t TW_SPIN_LIMIT = 1u << 20;           // default polls before a wait gives up

// Status bits raised by kernels of this library on the current device, read
// and cleared by la_device_status.
__device__ uint32_t la_dev_status;

// Per-row state in the workspace, zeroed before each launch.
struct TwRowState {
  uint32_t err;              // set when a bounded wait ran out
  uint32_t cnt[TW_PASSES];   // keys counted into each pass's histogram so far
  uint32_t pad[63 - TW_PASSES];
  uint32_t hist[TW_PASSES][TW_BINS];
};

struct TwKP {
  TopkKParams p;
  TwRowState *state;  // rows of this launch
  uint64_t *slots;    // [row of this launch][C]: (eq + 1) << 32 | gt once published
  double *cand_sc;    // order 0: candidate rows (NG x k) for the final sort
  int32_t *cand_id;
  int32_t *row_err;   // [NG]: set when a wait of the row ran out
  int64_t row0, C;
  uint32_t spin_limit;
  uint32_t unreachable;  // fault injection: no wait can ever be satisfied
};

__device__ __forceinline__ uint32_t tw_load(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tw_load64(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(TK_NT) void topk_wide_kernel(TwKP a) {
  __shared__ uint32_t hist[TW_BINS];
  __shared__ uint32_t eqc[TW_KPT][TK_NW];  // keys equal to the threshold, per slot and wave
  __shared__ uint32_t tkc[TW_KPT][TK_NW];  // keys taken, per slot and wave
  __shared__ uint32_t wtmp[2][TK_NW];
  __shared__ uint32_t s_bin, s_above, s_cnt;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint64_t lt = lanemask_lt(lane);
  const TopkKParams &p = a.p;
  const int64_t c = blockIdx.x, rl = blockIdx.y, gi = a.row0 + rl;
  const TkRow rw = tk_row(p, gi);
  TwRowState *st = a.state + rl;
  uint64_t *slots = a.slots + rl * a.C;
  const int64_t n_v = rw.n_v;
  const uint32_t K = (uint32_t)rw.K;
  const int64_t c0 = c * TW_CHUNK + tid;
  const double *rp = p.scores + rw.br * p.row_stride;

  uint64_t u[TW_KPT];
  {
    double v[TW_KPT];
#pragma unroll
    for (int j = 0; j < TW_KPT; ++j) {
      const int64_t i = c0 + (int64_t)j * TK_NT;
      v[j] = i < n_v ? rp[i] : 0.0;
    }
#pragma unroll
    for (int j = 0; j < TW_KPT; ++j) u[j] = ord_key(v[j]);
  }
  auto valid = [&](int j) { return c0 + (int64_t)j * TK_NT < n_v; };

  uint64_t prefix = 0, mask = 0;
  uint32_t need = K;
  bool all_in = (int64_t)K >= n_v;
  uint32_t expect = (uint32_t)n_v;  // keys of the row matching the prefix
  const uint32_t bump = a.unreachable;
  auto give_up = [&]() {
    __hip_atomic_store(&st->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&a.row_err[gi], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  int top = 63;
  for (int pass = 0; !all_in && top >= 0; ++pass) {
    const int shift = top >= TW_RB - 1 ? top - (TW_RB - 1) : 0;
    const uint32_t dm = (2u << (top - shift)) - 1u;
    for (int b = tid; b < TW_BINS; b += TK_NT) hist[b] = 0u;
    __syncthreads();
    uint32_t mine = 0;  // keys of this thread the pass counts
#pragma unroll
    for (int j = 0; j < TW_KPT; ++j) {
      if (valid(j) && (u[j] & mask) == prefix) {
        atomicAdd(&hist[(uint32_t)(u[j] >> shift) & dm], 1u);
        ++mine;
      }
    }
    __syncthreads();
    uint32_t *gh = st->hist[pass];
    for (int b = tid; b < TW_BINS; b += TK_NT) {
      const uint32_t x = hist[b];
      if (x) __hip_atomic_fetch_add(&gh[b], x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    tk_block_incl_scan(mine, wtmp[1], mine);
    if (tid == 0 && mine)
      __hip_atomic_fetch_add(&st->cnt[pass], mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Wait (one thread) until the row's running count shows every chunk's
    // keys, then read the row's histogram until its bins sum to the same
    // number: bins only grow, so such a read saw every bin's final count.
    // Thread t holds bins TW_BINS - 1 - TW_BPT * t downwards.
    if (tid == 0) {
      for (uint32_t spins = 0; tw_load(&st->cnt[pass]) < expect + bump && spins < a.spin_limit;
           ++spins)
        __builtin_amdgcn_s_sleep(2);
    }
    __syncthreads();
    uint32_t h[TW_BPT], csum, incl, tot;
    for (uint32_t spins = 0;; ++spins) {
      csum = 0;
#pragma unroll
      for (int e = 0; e < TW_BPT; ++e) {
        h[e] = tw_load(&gh[TW_BINS - 1 - TW_BPT * tid - e]);
        csum += h[e];
      }
      incl = tk_block_incl_scan(csum, wtmp[0], tot);
      if (tot == expect + bump) break;
      if (spins >= a.spin_limit) {
        if (tid == 0) give_up();
        return;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    // the bin holding the need-th largest key
    if (incl >= need && incl - csum < need) {
      uint32_t acc = incl - csum;
      bool found = false;
#pragma unroll
      for (int e = 0; e < TW_BPT; ++e) {
        if (!found && acc + h[e] >= need) {
          s_bin = (uint32_t)(TW_BINS - 1 - TW_BPT * tid - e);
          s_above = acc;
          s_cnt = h[e];
          found = true;
        }
        acc += h[e];
      }
    }
    __syncthreads();
    need -= s_above;
    prefix |= (uint64_t)s_bin << shift;
    mask |= (uint64_t)dm << shift;
    all_in = s_cnt == need;
    expect = s_cnt;
    __syncthreads();
    top = shift - 1;
  }

  // this chunk's keys above and equal to the threshold, published for the
  // chunks after it
  uint32_t gt = 0, eq = 0;
#pragma unroll
  for (int j = 0; j < TW_KPT; ++j) {
    const uint64_t um = u[j] & mask;
    gt += valid(j) && um > prefix;
    eq += valid(j) && um == prefix;
  }
  uint32_t gt_c, eq_c;
  tk_block_incl_scan(gt, wtmp[0], gt_c);
  tk_block_incl_scan(eq, wtmp[1], eq_c);
  if (tid == 0)
    __hip_atomic_store(&slots[c], ((uint64_t)(eq_c + 1) << 32) | gt_c, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  // counts of the chunks before this one
  uint32_t gb = 0, eb = 0, bad = 0;
  for (int64_t x = tid; x < c; x += TK_NT) {
    uint64_t v = bump ? 0 : tw_load64(&slots[x]);
    uint32_t spins = 0;
    while (v == 0 && ++spins <= a.spin_limit) {
      __builtin_amdgcn_s_sleep(2);
      v = bump ? 0 : tw_load64(&slots[x]);
    }
    if (v == 0) {
      bad = 1;
      give_up();
    } else {
      gb += (uint32_t)v;
      eb += (uint32_t)(v >> 32) - 1u;
    }
  }
  uint32_t gt_before, eq_before, n_bad;
  tk_block_incl_scan(gb, wtmp[0], gt_before);
  tk_block_incl_scan(eb, wtmp[1], eq_before);
  tk_block_incl_scan(bad, wtmp[0], n_bad);
  if (n_bad) return;
  const uint32_t sel_before = gt_before + (all_in ? eq_before : min(need, eq_before));

  // ranks of the threshold keys (index order), then the taken keys' slots
  if (!all_in) {
#pragma unroll
    for (int j = 0; j < TW_KPT; ++j) {
      const uint64_t b = __ballot(valid(j) && (u[j] & mask) == prefix);
      if (lane == 0) eqc[j][w] = (uint32_t)__popcll(b);
    }
    __syncthreads();
  }
  uint32_t take_bits = 0, eq_run = eq_before;
#pragma unroll
  for (int j = 0; j < TW_KPT; ++j) {
    const uint64_t um = u[j] & mask;
    const bool is_gt = valid(j) && um > prefix;
    const bool is_eq = valid(j) && um == prefix;
    bool take = is_gt || (is_eq && all_in);
    if (!all_in) {
      const uint64_t b = __ballot(is_eq);
      uint32_t rank = eq_run + (uint32_t)__popcll(b & lt);
#pragma unroll
      for (int x = 0; x < TK_NW; ++x) rank += x < w ? eqc[j][x] : 0u;
      take = is_gt || (is_eq && rank < need);
#pragma unroll
      for (int x = 0; x < TK_NW; ++x) eq_run += eqc[j][x];
    }
    const uint64_t tb = __ballot(take);
    if (lane == 0) tkc[j][w] = (uint32_t)__popcll(tb);
    take_bits |= (uint32_t)take << j;
  }
  __syncthreads();
  const bool ord1 = p.order == 1;
  int32_t *oi = p.out_idx + rw.orow * p.width;
  uint32_t pos_run = sel_before;
#pragma unroll
  for (int j = 0; j < TW_KPT; ++j) {
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
  const int64_t stride = a.C * TK_NT;
  if (ord1) {
    for (int64_t x = K + c * TK_NT + tid; x < p.width; x += stride) oi[x] = -1;
    if (c == 0 && tid == 0 && p.out_count)
      p.out_count[rw.orow] = (int32_t)min((int64_t)K, p.width);
  } else {
    // the lowest key (all-ones pattern) and index -1: sorted after every real one
    for (int64_t x = K + c * TK_NT + tid; x < p.k; x += stride) {
      a.cand_sc[gi * p.k + x] = __longlong_as_double((long long)0xffffffffffffffffull);
      a.cand_id[gi * p.k + x] = -1;
    }
  }
}

__global__ __launch_bounds__(256) void tw_clear_kernel(uint4 *p, int64_t n16) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// After every batch (and the sort of a sorted selection): rows whose wait ran
// out get -1 ids, -inf values and count -1, and the device status word
// records the timeout.  One workgroup per row.
__global__ __launch_bounds__(256) void tw_finish_kernel(TopkKParams p, const int32_t *row_err) {
  const int64_t gi = blockIdx.x;
  if (row_err[gi] == 0) return;
  const TkRow rw = tk_row(p, gi);
  int32_t *oi = p.out_idx + rw.orow * p.width;
  for (int64_t x = threadIdx.x; x < p.width; x += 256) oi[x] = -1;
  if (p.out_val)
    for (int64_t x = threadIdx.x; x < p.width; x += 256)
      p.out_val[rw.orow * p.width + x] = __int_as_float(0xff800000);
  if (threadIdx.x == 0) {
    if (p.out_count) p.out_count[rw.orow] = -1;
    __hip_atomic_fetch_or(&la_dev_status, (uint32_t)LA_DEV_TOPK_TIMEOUT, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
  }
}

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// Workgroups of the wide kernel one device holds at once (0: no cooperative
// launch there).
static int64_t wide_capacity() {
  static int64_t cached = -1;
  static int cached_dev = -1;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (cached >= 0 && cached_dev == dev) return cached;
  int coop = 0, per_cu = 0;
  int64_t cap = 0;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) == hipSuccess &&
      coop &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, topk_wide_kernel, TK_NT, 0) ==
          hipSuccess)
    cap = (int64_t)per_cu * num_cus();
  cached = cap;
  cached_dev = dev;
  return cap;
}

WidePlan wide_plan(const TopkKParams &p) {
  WidePlan W;
  // LA_TOPK_WIDE=0 keeps long rows on the segmented levels (kept for devices
  // without cooperative launch, and tested against the same oracle)
  const char *env = getenv("LA_TOPK_WIDE");
  if (env && env[0] == '0') return W;
  W.plain = env && strcmp(env, "plain") == 0;
  const int64_t cap = wide_capacity();
  W.C = ceil_div(p.n, TW_CHUNK);
  if (cap <= 0 || W.C > cap || p.n >= ((int64_t)1 << 31)) {
    W.C = 0;
    return W;
  }
  W.R = std::min(p.NG, cap / W.C);
  W.state_bytes = align256(W.R * (int64_t)sizeof(TwRowState)) + align256(W.R * W.C * 8);
  W.bytes = W.state_bytes + align256(p.NG * 4);
  if (p.order == 0) W.bytes += align256(p.NG * p.k * 8) + align256(p.NG * p.k * 4);
  return W;
}

int topk_wide_launch(const TopkKParams &p, const WidePlan &W, void *ws, hipStream_t st) {
  if ((uintptr_t)ws % 16 != 0) return fail(LA_ERR_INVALID, "topk: workspace not 16-byte aligned");
  char *base = (char *)ws;
  TwKP a{};
  a.p = p;
  a.state = (TwRowState *)base;
  a.slots = (uint64_t *)(base + align256(W.R * (int64_t)sizeof(TwRowState)));
  a.C = W.C;
  a.row_err = (int32_t *)(base + W.state_bytes);
  const int64_t err_bytes = align256(p.NG * 4);
  if (p.order == 0) {
    a.cand_sc = (double *)(base + W.state_bytes + err_bytes);
    a.cand_id = (int32_t *)(base + W.state_bytes + err_bytes + align256(p.NG * p.k * 8));
  }
  // wait limits: LA_TOPK_WIDE_SPIN polls (default 2^20); LA_TOPK_WIDE_FAULT=1
  // makes every wait unsatisfiable (tests of the timeout path)
  a.spin_limit = TW_SPIN_LIMIT;
  if (const char *e = getenv("LA_TOPK_WIDE_SPIN")) a.spin_limit = (uint32_t)strtoul(e, nullptr, 10);
  if (const char *e = getenv("LA_TOPK_WIDE_FAULT")) a.unreachable = e[0] == '1' ? 1u : 0u;
  // the row flags once, then the state of each batch
  {
    const int64_t n16 = (W.state_bytes + err_bytes) / 16;
    tw_clear_kernel<<<(unsigned)std::min<int64_t>(ceil_div(n16, 256), 1024), 256, 0, st>>>(
        (uint4 *)base, n16);
    LA_LAUNCHED();
  }
  const int64_t n16 = W.state_bytes / 16;
  const unsigned clear_grid = (unsigned)std::min<int64_t>(ceil_div(n16, 256), 1024);
  for (int64_t row0 = 0; row0 < p.NG; row0 += W.R) {
    const int64_t rows = std::min(W.R, p.NG - row0);
    if (row0 > 0) {
      tw_clear_kernel<<<clear_grid, 256, 0, st>>>((uint4 *)base, n16);
      LA_LAUNCHED();
    }
    a.row0 = row0;
    const dim3 grid((unsigned)W.C, (unsigned)rows);
    if (W.plain) {
      // LA_TOPK_WIDE=plain: an ordinary launch of the same grid (it fits the
      // device at once, but residency is not guaranteed: a wait that runs out
      // is reported as above).  For profilers that cannot follow a
      // cooperative launch.
      topk_wide_kernel<<<grid, TK_NT, 0, st>>>(a);
      LA_LAUNCHED();
    } else {
      void *args[] = {&a};
      LA_HIP(hipLaunchCooperativeKernel((const void *)topk_wide_kernel, grid, dim3(TK_NT), args,
                                        0, st));
    }
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
  tw_finish_kernel<<<dim3((unsigned)p.NG), 256, 0, st>>>(p, a.row_err);
  LA_LAUNCHED();
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
