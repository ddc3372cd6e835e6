/*
 * CPU oracle for the MLA decode path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is a checker: only tests/, the smoke
 * entry point and the CPU-baseline leg of the benchmark may load it. The
 * product path (triton_mla.mla_decode) never calls it and has no CPU
 * fallback.
 *
 * It restates, in plain C with float64 arithmetic, the reference's PyTorch
 * oracles and its split heuristic:
 *   - gather_kv            src/triton_mla/reference.py:6-13
 *   - mla_decode_ref       src/triton_mla/reference.py:16-31
 *   - get_num_splits       src/triton_mla/kernel.py:190-201
 *   - the stage-1/stage-2 split-and-merge algebra of the fused kernel,
 *     kernel.py:83-86 (split ranges), 119-128 (online softmax + guards),
 *     165-181 (log-sum-exp merge), used to pin split invariance.
 *
 * Pins (see tests/test_oracle.py):
 *   gather_kv          bit-exact against torch indexing of the same cache and
 *                      against paged/dense equivalence.
 *   mla_decode_ref     closed forms (one token: out == latent row; zero query:
 *                      out == mean of latent rows, lse == log n), scipy's
 *                      softmax/logsumexp on random inputs, brute force on tiny
 *                      inputs, token-permutation invariance.
 *   get_num_splits     the 16-row known-answer table in results/bench_h100.csv.
 *   split_merge        equals mla_decode_ref for every split count.
 *
 * Element types: 0 = bfloat16, 1 = float16 (raw 16-bit patterns).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_BF16 0
#define ORACLE_FP16 1

/* Exact widening of a 16-bit float pattern. */
static double half_bits_to_double(uint16_t h, int dtype) {
    if (dtype == ORACLE_BF16) {
        uint32_t u = ((uint32_t)h) << 16;
        float f;
        memcpy(&f, &u, 4);
        return (double)f;
    }
    /* IEEE binary16 */
    uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    double v;
    if (exp == 0)
        v = ldexp((double)man, -24);
    else if (exp == 31)
        v = man ? NAN : INFINITY;
    else
        v = ldexp((double)(man | 0x400u), (int)exp - 25);
    return sign ? -v : v;
}

double oracle_half_to_double(uint16_t h, int dtype) { return half_bits_to_double(h, dtype); }

/* Round-to-nearest-even narrowing of a float32 value to a 16-bit pattern. */
uint16_t oracle_float_to_half_bits(float f, int dtype) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if (dtype == ORACLE_BF16) {
        if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
        uint32_t lsb = (u >> 16) & 1u;
        u += 0x7fffu + lsb;
        return (uint16_t)(u >> 16);
    }
    /* float32 -> binary16, round to nearest even, via double arithmetic */
    double d = (double)f;
    uint16_t sign = (uint16_t)((u >> 31) << 15);
    if (isnan(d)) return (uint16_t)(sign | 0x7e00u);
    double a = fabs(d);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7c00u);
    if (a < ldexp(1.0, -14)) { /* subnormal range: quantum 2^-24 */
        double q = nearbyint(a * ldexp(1.0, 24));
        return (uint16_t)(sign | (uint16_t)q);
    }
    int e;
    double m = frexp(a, &e); /* a = m * 2^e, m in [0.5, 1) */
    double q = nearbyint(m * 2048.0); /* 11 significant bits */
    if (q >= 2048.0) { q /= 2.0; e += 1; }
    uint16_t exp_field = (uint16_t)(e - 1 + 15);
    return (uint16_t)(sign | (exp_field << 10) | ((uint16_t)q & 0x3ffu));
}

void oracle_round_to_half(const float* in, uint16_t* out, int64_t n, int dtype) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_float_to_half_bits(in[i], dtype);
}

/*
 * Address (in elements) of token t of sequence b.
 * Paged: kv[bt[b, t / page_size], t % page_size]; dense: kv[b, t].
 * Follows gather_kv, reference.py:6-13 (kv_cache[block_table].reshape(B, -1, D)).
 */
static int64_t token_offset(int64_t b, int64_t t, const int32_t* bt, int64_t bt_s0, int paged,
                            int64_t page_size, int64_t kv_s0, int64_t kv_s1) {
    if (paged) {
        int64_t page = bt[b * bt_s0 + t / page_size];
        return page * kv_s0 + (t % page_size) * kv_s1;
    }
    return b * kv_s0 + t * kv_s1;
}

/*
 * gather_kv (reference.py:6-13): out[b, t, :] = cache row of token t of
 * sequence b, for t in [0, n_tokens). Bit-exact copy of 16-bit patterns.
 */
void oracle_gather_kv(const uint16_t* kv, int64_t kv_s0, int64_t kv_s1, const int32_t* bt,
                      int64_t bt_s0, int paged, int64_t page_size, int64_t batch,
                      int64_t n_tokens, int64_t d, uint16_t* out) {
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t t = 0; t < n_tokens; ++t)
            memcpy(out + (b * n_tokens + t) * d,
                   kv + token_offset(b, t, bt, bt_s0, paged, page_size, kv_s0, kv_s1),
                   (size_t)d * 2);
}

/*
 * mla_decode_ref (reference.py:16-31), float64 throughout:
 *   s = q[b] . k^T * scale;  lse = logsumexp(s);  out = softmax(s) . k[:, :dv]
 *   n == 0  =>  out = 0, lse = -inf.
 * q is [B, H, dqk] with element strides (q_sb, q_sh, 1). out is float32
 * [B, H, dv] (not rounded: the caller rounds to the input dtype), lse is
 * float32 [B, H] natural log.
 */
int oracle_mla_decode_ref(const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint16_t* kv,
                          int64_t kv_s0, int64_t kv_s1, const int32_t* bt, int64_t bt_s0,
                          int paged, int64_t page_size, const int32_t* seqlens, int64_t batch,
                          int64_t heads, int64_t dqk, int64_t dv, int dtype, double scale,
                          int nthreads, float* out, float* lse) {
    if (dv > dqk || dqk <= 0 || heads < 0 || batch < 0) return 1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    for (int64_t b = 0; b < batch; ++b) {
        const int64_t n = seqlens[b];
        if (n <= 0) {
            for (int64_t h = 0; h < heads; ++h) {
                lse[b * heads + h] = -INFINITY;
                for (int64_t c = 0; c < dv; ++c) out[(b * heads + h) * dv + c] = 0.0f;
            }
            continue;
        }
        double* k = (double*)malloc((size_t)(n * dqk) * sizeof(double));
        if (!k) return 2;
#pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < n; ++t) {
            const uint16_t* row = kv + token_offset(b, t, bt, bt_s0, paged, page_size, kv_s0, kv_s1);
            for (int64_t c = 0; c < dqk; ++c) k[t * dqk + c] = half_bits_to_double(row[c], dtype);
        }
        int failed = 0;
#pragma omp parallel
        {
            double* s = (double*)malloc((size_t)n * sizeof(double));
            double* qd = (double*)malloc((size_t)dqk * sizeof(double));
            double* acc = (double*)malloc((size_t)dv * sizeof(double));
            if (!s || !qd || !acc) {
#pragma omp atomic write
                failed = 1;
            } else {
#pragma omp for schedule(dynamic, 1)
                for (int64_t h = 0; h < heads; ++h) {
                    const uint16_t* qr = q + b * q_sb + h * q_sh;
                    for (int64_t c = 0; c < dqk; ++c) qd[c] = half_bits_to_double(qr[c], dtype);
                    double m = -INFINITY;
                    for (int64_t t = 0; t < n; ++t) {
                        const double* kr = k + t * dqk;
                        double dot = 0.0;
                        for (int64_t c = 0; c < dqk; ++c) dot += qd[c] * kr[c];
                        s[t] = dot * scale;
                        if (s[t] > m) m = s[t];
                    }
                    double l = 0.0;
                    for (int64_t c = 0; c < dv; ++c) acc[c] = 0.0;
                    for (int64_t t = 0; t < n; ++t) {
                        const double p = exp(s[t] - m);
                        const double* kr = k + t * dqk;
                        l += p;
                        for (int64_t c = 0; c < dv; ++c) acc[c] += p * kr[c];
                    }
                    lse[b * heads + h] = (float)(m + log(l));
                    for (int64_t c = 0; c < dv; ++c) out[(b * heads + h) * dv + c] = (float)(acc[c] / l);
                }
            }
            free(s);
            free(qd);
            free(acc);
        }
        free(k);
        if (failed) return 2;
    }
    return 0;
}

/*
 * get_num_splits (kernel.py:190-201): largest power of two <=
 * max(min(num_sms // max(batch * cdiv(heads, 64), 1), cdiv(max_seqlen, min_tokens), 64), 1).
 */
int64_t oracle_get_num_splits(int64_t batch, int64_t heads, int64_t max_seqlen, int64_t num_sms,
                              int64_t min_tokens_per_split) {
    int64_t head_groups = (heads + 63) / 64;
    int64_t denom = batch * head_groups;
    if (denom < 1) denom = 1;
    int64_t target = num_sms / denom;
    int64_t max_by_len = (max_seqlen + min_tokens_per_split - 1) / min_tokens_per_split;
    int64_t s = target < max_by_len ? target : max_by_len;
    if (s > 64) s = 64;
    if (s < 1) s = 1;
    int64_t p = 1;
    while (p * 2 <= s) p *= 2;
    return p;
}

/*
 * The fused kernel's split/merge algebra (kernel.py:83-86, 119-128, 165-181),
 * restated in float64 for one (b, h): the sequence is cut into num_splits
 * ranges of cdiv(n, num_splits) tokens, each range yields a normalised partial
 * and a base-2 log-sum-exp (-inf and a zero partial when empty), and the merge
 * weights partials by 2^(lse_s - max). Writes the merged out[dv] and the
 * natural-log lse. Used only to show that splitting does not change the
 * result.
 */
int oracle_split_merge(const uint16_t* q, const uint16_t* kv, int64_t kv_s0, int64_t kv_s1,
                       const int32_t* bt, int64_t bt_s0, int paged, int64_t page_size,
                       int64_t b, int64_t n, int64_t dqk, int64_t dv, int dtype, double scale,
                       int64_t num_splits, float* out, float* lse_out) {
    const double log2e = 1.4426950408889634, ln2 = 0.6931471805599453;
    if (num_splits < 1) return 1;
    double* po = (double*)calloc((size_t)(num_splits * dv), sizeof(double));
    double* plse = (double*)malloc((size_t)num_splits * sizeof(double));
    double* acc = (double*)malloc((size_t)dv * sizeof(double));
    if (!po || !plse || !acc) { free(po); free(plse); free(acc); return 2; }
    const int64_t split_len = (n + num_splits - 1) / num_splits;
    for (int64_t s = 0; s < num_splits; ++s) {
        int64_t start = s * split_len, end = start + split_len;
        if (end > n) end = n;
        double m = -INFINITY, l = 0.0;
        for (int64_t c = 0; c < dv; ++c) acc[c] = 0.0;
        for (int64_t t = start; t < end; ++t) {
            const uint16_t* row = kv + token_offset(b, t, bt, bt_s0, paged, page_size, kv_s0, kv_s1);
            double dot = 0.0;
            for (int64_t c = 0; c < dqk; ++c) dot += half_bits_to_double(q[c], dtype) * half_bits_to_double(row[c], dtype);
            const double x = dot * scale * log2e;
            const double m_new = x > m ? x : m;
            const double alpha = exp2(m - m_new), p = exp2(x - m_new);
            l = l * alpha + p;
            for (int64_t c = 0; c < dv; ++c) acc[c] = acc[c] * alpha + p * half_bits_to_double(row[c], dtype);
            m = m_new;
        }
        if (l > 0) {
            for (int64_t c = 0; c < dv; ++c) po[s * dv + c] = acc[c] / l;
            plse[s] = m + log2(l);
        } else {
            plse[s] = -INFINITY;
        }
    }
    double mx = -INFINITY;
    for (int64_t s = 0; s < num_splits; ++s) if (plse[s] > mx) mx = plse[s];
    if (mx == -INFINITY) mx = 0.0;
    double wsum = 0.0;
    for (int64_t c = 0; c < dv; ++c) acc[c] = 0.0;
    for (int64_t s = 0; s < num_splits; ++s) {
        const double w = exp2(plse[s] - mx);
        for (int64_t c = 0; c < dv; ++c) acc[c] += w * po[s * dv + c];
        wsum += w;
    }
    for (int64_t c = 0; c < dv; ++c) out[c] = (float)(wsum > 0 ? acc[c] / wsum : 0.0);
    *lse_out = wsum > 0 ? (float)((mx + log2(wsum)) * ln2) : -INFINITY;
    free(po);
    free(plse);
    free(acc);
    return 0;
}
