/*
 * CPU oracle for the sparse-attention hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Nothing in the product links or calls this file.  It is loaded by tests/,
 * by __graft_entry__.smoke() (as the checker) and by bench.py's cpu_baseline
 * leg.  It restates, in plain C99, the arithmetic whose exact bits decide which
 * pages / blocks / tokens are selected, so that GPU selections can be compared
 * bit for bit:
 *
 *   or_quest_scores   quest_pages.py:51-55, selection.py:203-212
 *   or_topk_rows      selection.py:51-59 (topk_blocks), quest_pages.py:58-78,
 *                     fused_indexer.py:63-73 -- ties to the lowest index
 *   or_indexer_scores fused_indexer.py:52-60 (and selection.py:717-737)
 *   or_mean_pool      core.py:102-120 (block_reduce, mean, tail repeats last row)
 *   or_dot_rows       selection.py:339-345 (pooled q . pooled k block scores)
 *   or_sparse_attend  block_sparse.py:40-75, decode_attn.c:39-65 (gather + softmax)
 *   or_exp_det        a deterministic exp (fixed fma sequence) for XAttention
 *   or_xattn_select   selection.py:528-595 (antidiagonal scores, cumulative
 *                     mass threshold or top-k over integer block masses)
 *
 * Canonical arithmetic (the selection contract the HIP kernels reproduce):
 *   - inputs are fp32 / bf16 values widened exactly to fp64;
 *   - a product of two such values is exact in fp64, so sum_d x_d*y_d is
 *     accumulated in increasing d with one rounding per add;
 *   - products that are not exact (pooled means, indexer head weights) are
 *     rounded, then added -- never fused (built with -ffp-contract=off);
 *   - ranking is by value descending, ties to the lowest index, -0 == +0.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ scores ---- */

/* q: [R][G][D], mn/mx: [R][P][D] -> out [R][G][P].
 * score = sum_d max(q_d*mn_d, q_d*mx_d), d increasing. */
void or_quest_scores(const double *q, const double *mn, const double *mx, int64_t R, int64_t G,
                     int64_t P, int64_t D, double *out) {
  for (int64_t r = 0; r < R; ++r)
    for (int64_t g = 0; g < G; ++g) {
      const double *qv = q + (r * G + g) * D;
      for (int64_t p = 0; p < P; ++p) {
        const double *lo = mn + (r * P + p) * D;
        const double *hi = mx + (r * P + p) * D;
        double acc = 0.0;
        for (int64_t d = 0; d < D; ++d) {
          const double a = qv[d] * lo[d];
          const double b = qv[d] * hi[d];
          acc = acc + (a > b ? a : b);
        }
        out[(r * G + g) * P + p] = acc;
      }
    }
}

/* q: [Tq][HI][d], k: [Tk][HI][d], w: [Tq][HI] -> out [Tq][Tk];
 * only keys s < n_keys(t) = (causal_off >= 0 ? min(Tk, causal_off + t + 1) : Tk)
 * are written.  I = sum_h fl(w_h * relu(sum_e q_e*k_e)), h increasing. */
void or_indexer_scores(const double *q, const double *k, const double *w, int64_t Tq, int64_t Tk,
                       int64_t HI, int64_t d, int64_t causal_off, double *out) {
  for (int64_t t = 0; t < Tq; ++t) {
    int64_t nk = Tk;
    if (causal_off >= 0 && causal_off + t + 1 < nk) nk = causal_off + t + 1;
    for (int64_t s = 0; s < nk; ++s) {
      double acc = 0.0;
      for (int64_t h = 0; h < HI; ++h) {
        const double *qv = q + (t * HI + h) * d;
        const double *kv = k + (s * HI + h) * d;
        double dot = 0.0;
        for (int64_t e = 0; e < d; ++e) dot = dot + qv[e] * kv[e];
        const double r = dot > 0.0 ? dot : 0.0;
        const double wr = w[t * HI + h] * r;
        acc = acc + wr;
      }
      out[t * Tk + s] = acc;
    }
  }
}

/* x: [T][D] -> out [ceil(T/bs)][D]; mean over bs rows, tail padded with the
 * last row; rows summed in order, then divided by bs. */
void or_mean_pool(const double *x, int64_t T, int64_t D, int64_t bs, double *out) {
  const int64_t nb = (T + bs - 1) / bs;
  for (int64_t blk = 0; blk < nb; ++blk)
    for (int64_t dd = 0; dd < D; ++dd) {
      double acc = 0.0;
      for (int64_t i = 0; i < bs; ++i) {
        int64_t row = blk * bs + i;
        if (row > T - 1) row = T - 1;
        acc = acc + x[row * D + dd];
      }
      out[blk * D + dd] = acc / (double)bs;
    }
}

/* a: [Ra][D], b: [Rb][D] -> out [Ra][Rb], out = sum_d fl(a_d*b_d), d increasing. */
void or_dot_rows(const double *a, const double *b, int64_t Ra, int64_t Rb, int64_t D, double *out) {
  for (int64_t i = 0; i < Ra; ++i)
    for (int64_t j = 0; j < Rb; ++j) {
      double acc = 0.0;
      for (int64_t dd = 0; dd < D; ++dd) {
        const double pr = a[i * D + dd] * b[j * D + dd];
        acc = acc + pr;
      }
      out[i * Rb + j] = acc;
    }
}

/* ------------------------------------------------------------- top-k ---- */

typedef struct {
  double v;
  int32_t i;
  int32_t forced;
} or_item;

static int or_cmp(const void *pa, const void *pb) {
  const or_item *a = (const or_item *)pa, *b = (const or_item *)pb;
  if (a->forced != b->forced) return a->forced ? -1 : 1;
  if (!a->forced) {
    if (a->v > b->v) return -1;
    if (a->v < b->v) return 1;
  }
  return (a->i < b->i) ? -1 : (a->i > b->i);
}

/* scores [R][n]; row r considers i < n_valid[r]; own[r] (if force_own and in
 * range) ranks first.  Writes min(k, valid) indices sorted by (value desc,
 * index asc) to out_idx [R][k], -1 padded; out_val (optional) gets the values
 * (+inf for the forced entry), -inf padded.  Returns 0, or -1 on malloc failure. */
int or_topk_rows(const double *scores, int64_t R, int64_t n, const int32_t *n_valid,
                 const int32_t *own, int force_own, int64_t k, int32_t *out_idx, double *out_val) {
  or_item *items = (or_item *)malloc(sizeof(or_item) * (size_t)(n > 0 ? n : 1));
  if (!items) return -1;
  for (int64_t r = 0; r < R; ++r) {
    int64_t nv = n_valid ? n_valid[r] : n;
    if (nv > n) nv = n;
    if (nv < 0) nv = 0;
    const int64_t o = own ? own[r] : -1;
    for (int64_t i = 0; i < nv; ++i) {
      items[i].v = scores[r * n + i];
      items[i].i = (int32_t)i;
      items[i].forced = force_own && i == o;
    }
    qsort(items, (size_t)nv, sizeof(or_item), or_cmp);
    const int64_t kk = nv < k ? nv : k;
    for (int64_t j = 0; j < k; ++j) {
      out_idx[r * k + j] = j < kk ? items[j].i : -1;
      if (out_val)
        out_val[r * k + j] = j < kk ? (items[j].forced ? INFINITY : items[j].v) : -INFINITY;
    }
  }
  free(items);
  return 0;
}

/* ------------------------------------------------------- attention ---- */

/* Element readers for the KV cache: 0 = fp32, 1 = bf16 (uint16 bits),
 * 3 = fp8 e4m3fn code (uint8) times a per-token scale. */
static double or_bf16(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return (double)f;
}

/* OCP FP8 E4M3FN: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities,
 * S.1111.111 is NaN; subnormals are m * 2^-9. */
double or_fp8_e4m3fn(uint8_t c) {
  const int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
  double v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0)
    v = ldexp((double)m, -9);
  else
    v = ldexp(1.0 + m / 8.0, e - 7);
  return s ? -v : v;
}

static double or_load(const void *base, int64_t idx, int dt) {
  switch (dt) {
    case 0: return (double)((const float *)base)[idx];
    case 1: return or_bf16(((const uint16_t *)base)[idx]);
    case 3: return or_fp8_e4m3fn(((const uint8_t *)base)[idx]);
    default: return 0.0;
  }
}

/* Exact attention of one query row over a token list (fp64 throughout).
 *   q: [G][D] (fp64) for the G query heads sharing the list
 *   kv addressing: contiguous (page_table == NULL): element offset of token
 *     tok = tok*st; paged: page_table[tok/ps] -> ((phys*Hkv + kvh)*ps + tok%ps)*D.
 *   toks: n_tok logical token indices (already expanded from unit ids; -1 skipped)
 *   out: [G][D] fp64; an empty list gives zeros.
 * Scores are q.k * scale; softmax subtracts the max.  Returns 0. */
int or_sparse_attend(const double *q, int64_t G, int64_t D, const void *k, const void *v, int dt,
                     const float *k_scale, const float *v_scale, const int32_t *page_table,
                     int64_t ps, int64_t Hkv, int64_t kvh, int64_t k_st, int64_t v_st,
                     int64_t s_st, const int64_t *toks, int64_t n_tok, double scale, double *out,
                     double *work /* [n_tok] */) {
  for (int64_t g = 0; g < G; ++g) {
    const double *qv = q + g * D;
    double mx = -INFINITY;
    int64_t valid = 0;
    for (int64_t j = 0; j < n_tok; ++j) {
      const int64_t tok = toks[j];
      if (tok < 0) {
        work[j] = -INFINITY;
        continue;
      }
      int64_t ko, so;
      if (page_table) {
        const int64_t row = ((int64_t)page_table[tok / ps] * Hkv + kvh) * ps + tok % ps;
        ko = row * D;
        so = row;
      } else {
        ko = tok * k_st;
        so = tok * s_st;
      }
      double s = 0.0;
      for (int64_t d = 0; d < D; ++d) s += qv[d] * or_load(k, ko + d, dt);
      if (dt == 3) s *= (double)k_scale[so];
      s *= scale;
      work[j] = s;
      if (s > mx) mx = s;
      ++valid;
    }
    double *o = out + g * D;
    for (int64_t d = 0; d < D; ++d) o[d] = 0.0;
    if (!valid) continue;
    double l = 0.0;
    for (int64_t j = 0; j < n_tok; ++j) {
      const int64_t tok = toks[j];
      if (tok < 0) continue;
      const double p = exp(work[j] - mx);
      l += p;
      int64_t vo, so;
      if (page_table) {
        const int64_t row = ((int64_t)page_table[tok / ps] * Hkv + kvh) * ps + tok % ps;
        vo = row * D;
        so = row;
      } else {
        vo = tok * v_st;
        so = tok * s_st;
      }
      const double pv = (dt == 3) ? p * (double)v_scale[so] : p;
      for (int64_t d = 0; d < D; ++d) o[d] += pv * or_load(v, vo + d, dt);
    }
    for (int64_t d = 0; d < D; ++d) o[d] /= l;
  }
  return 0;
}

/* ------------------------------------------------------- XAttention ---- */

/* exp(x) for x <= 0 by a fixed sequence of correctly rounded operations, so
 * that csrc/xattn.hip (the same sequence) reproduces every bit: 0 below -700;
 * x = k*ln2 + r with the fdlibm two-part ln2 and fused multiply-adds; e^r by
 * the degree-13 Taylor polynomial in Horner form (fma); times 2^k built from
 * exponent bits. */
double or_exp_det(double x) {
  if (!(x > -700.0)) return 0.0;
  const double kf = nearbyint(x * 1.4426950408889634);
  double r = fma(-kf, 6.93147180369123816490e-01, x);
  r = fma(-kf, 1.90821492927058770002e-10, r);
  double p = 1.6059043836821613e-10;
  p = fma(p, r, 2.08767569878681e-09);
  p = fma(p, r, 2.505210838544172e-08);
  p = fma(p, r, 2.755731922398589e-07);
  p = fma(p, r, 2.7557319223985893e-06);
  p = fma(p, r, 2.48015873015873e-05);
  p = fma(p, r, 0.0001984126984126984);
  p = fma(p, r, 0.001388888888888889);
  p = fma(p, r, 0.008333333333333333);
  p = fma(p, r, 0.041666666666666664);
  p = fma(p, r, 0.16666666666666666);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  uint64_t bits = (uint64_t)((int64_t)kf + 1023) << 52;
  double two_k;
  memcpy(&two_k, &bits, 8);
  return p * two_k;
}

typedef struct {
  uint64_t mass;
  int64_t kb;
} or_mass_t;

static int or_mass_cmp(const void *pa, const void *pb) {
  const or_mass_t *a = (const or_mass_t *)pa, *b = (const or_mass_t *)pb;
  if (a->mass != b->mass) return a->mass > b->mass ? -1 : 1;
  return a->kb < b->kb ? -1 : (a->kb > b->kb);
}

/* XAttention.antidiagonal_scores + select (variants/selection.py:528-595)
 * for one (batch, query head): q [Tq][D] and the head's KV rows k [T][D]
 * (fp64 images of the inputs).  Blocks of blk tokens; slot s (antidiagonal
 * offset o = s*r <= 2*blk - 2, selection.py:554) = sum over i increasing of
 * the dot products q[qb*blk+i] . k[kb*blk+o-i] (fma over d increasing; rows
 * past Tq / T are zero rows, F.pad at :544-546), times inv_sqrt_d (:566).
 * Visible blocks: kb*blk <= qb*blk + offset (:573-575).  Weights
 * or_exp_det(slot - row max) as integers nearbyint(w * 2^F), F = 52 -
 * ceil(log2(n_kb*n_slots)); block mass = the sum over its slots (:576-579).
 * mode 0: blocks sorted by (mass desc, index asc), keep 1 + #{m : C_m <
 * ceil(alpha*Z)} (C_m prefix sums, Z the total; alpha*Z > Z keeps all;
 * _cumulative_select :62-69); mode 1: the first min(topk, n_kb) (:581-582).
 * Then the own block (first token qb*blk + offset) is OR'd in and invisible
 * blocks dropped (:591-592).  out [n_qb][width] ascending, -1 padded;
 * count [n_qb].  Returns 0, or -1 on a bad argument. */
int or_xattn_select(const double *q, const double *k, int64_t Tq, int64_t T, int64_t D,
                    int64_t blk, int64_t r, int64_t offset, double inv_sqrt_d, int mode,
                    double alpha, int64_t topk, int64_t width, int32_t *out, int32_t *count) {
  if (blk < 1 || r < 1 || Tq < 1 || T < 1 || D < 1 || offset < 0) return -1;
  const int64_t n_qb = (Tq + blk - 1) / blk, n_kb = (T + blk - 1) / blk;
  const int64_t ns = (2 * blk - 2) / r + 1;
  int64_t lg = 0;
  while (((int64_t)1 << lg) < n_kb * ns) ++lg;
  const double two_f = ldexp(1.0, (int)(52 - lg));
  double *S = (double *)malloc((size_t)(n_kb * ns) * sizeof(double));
  or_mass_t *m = (or_mass_t *)malloc((size_t)n_kb * sizeof(or_mass_t));
  unsigned char *keep = (unsigned char *)malloc((size_t)n_kb);
  if (!S || !m || !keep) {
    free(S);
    free(m);
    free(keep);
    return -1;
  }
  for (int64_t qb = 0; qb < n_qb; ++qb) {
    const int64_t pos0 = qb * blk + offset;
    int64_t lim = pos0 / blk;
    if (lim > n_kb - 1) lim = n_kb - 1;
    double mx = -INFINITY;
    for (int64_t kb = 0; kb <= lim; ++kb) {
      for (int64_t s = 0; s < ns; ++s) {
        const int64_t o = s * r;
        const int64_t i0 = o - blk + 1 > 0 ? o - blk + 1 : 0, i1 = o < blk - 1 ? o : blk - 1;
        double acc = 0.0;
        for (int64_t i = i0; i <= i1; ++i) {
          const int64_t qr = qb * blk + i, kr = kb * blk + (o - i);
          double e = 0.0;
          for (int64_t d = 0; d < D; ++d) {
            const double qv = qr < Tq ? q[qr * D + d] : 0.0;
            const double kv = kr < T ? k[kr * D + d] : 0.0;
            e = fma(qv, kv, e);
          }
          acc = acc + e;
        }
        S[kb * ns + s] = acc * inv_sqrt_d;
        if (S[kb * ns + s] > mx) mx = S[kb * ns + s];
      }
    }
    uint64_t Z = 0;
    for (int64_t kb = 0; kb < n_kb; ++kb) {
      uint64_t ms = 0;
      if (kb <= lim)
        for (int64_t s = 0; s < ns; ++s)
          ms += (uint64_t)nearbyint(or_exp_det(S[kb * ns + s] - mx) * two_f);
      m[kb].mass = ms;
      m[kb].kb = kb;
      Z += ms;
    }
    qsort(m, (size_t)n_kb, sizeof(or_mass_t), or_mass_cmp);
    int64_t n_keep;
    if (mode == 1) {
      n_keep = topk < n_kb ? topk : n_kb;
    } else {
      const double thr_d = alpha * (double)Z;
      if (thr_d > (double)Z) {
        n_keep = n_kb;
      } else {
        const uint64_t thr = thr_d > 0.0 ? (uint64_t)ceil(thr_d) : 0;
        uint64_t c = 0;
        n_keep = 1;
        for (int64_t i = 0; i < n_kb; ++i) {
          c += m[i].mass;
          if (c < thr) ++n_keep;
        }
        if (n_keep > n_kb) n_keep = n_kb;
      }
    }
    memset(keep, 0, (size_t)n_kb);
    for (int64_t i = 0; i < n_keep; ++i) keep[m[i].kb] = 1;
    if (pos0 % blk == 0 && pos0 / blk < n_kb) keep[pos0 / blk] = 1;
    int64_t c = 0;
    int32_t *o = out + qb * width;
    for (int64_t kb = 0; kb <= lim; ++kb)
      if (keep[kb]) {
        if (c < width) o[c] = (int32_t)kb;
        ++c;
      }
    for (int64_t i = c; i < width; ++i) o[i] = -1;
    count[qb] = (int32_t)(c < width ? c : width);
  }
  free(S);
  free(m);
  free(keep);
  return 0;
}
