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
 *   - an fp8 latent cache (no counterpart in the reference, whose README.md
 *     :32-33 lists "no FP8 cache"): OCP FP8 E4M3 ("e4m3fn") decoding and
 *     round-to-nearest-even encoding, and mla_decode_ref over the cache
 *     dequantised as e4m3(byte) * scale[page * s0 + row_in_page * s1].
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
 *   e4m3 decode        closed forms (0, 1, 448, 2^-9, 2^-6, NaN codes, sign
 *                      symmetry), monotonicity, and torch.float8_e4m3fn's
 *                      decoding of all 256 codes.
 *   e4m3 encode        decode-encode round trip of every code, tie cases
 *                      (to even mantissa), overflow to NaN above 464, and
 *                      torch's float32 -> float8_e4m3fn rounding on random
 *                      values.
 *   mla_decode_fp8_ref equals mla_decode_ref bit for bit on the same values
 *                      as a bf16 cache (power-of-two scales keep every
 *                      dequantised value a bf16 value), a numpy float64
 *                      softmax over the dequantised cache for arbitrary
 *                      per-token scales, and per-page == per-token scales
 *                      that repeat the page's value.
 *
 * Element types: 0 = bfloat16, 1 = float16 (raw 16-bit patterns), 2 =
 * float32 (mla_decode_ref only: q and the cache as float arrays; the
 * reference's kernels take any element type q and the cache share,
 * kernel.py:245). Pinned like the 16-bit types, and equal to them bit for
 * bit on values both can hold.
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
#define ORACLE_FP32 2

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
 * Attention of every head of sequence b over n rows k[t * dqk + c] (float64):
 *   s = q[b, h] . k^T * scale;  lse = logsumexp(s);  out = softmax(s) . k[:, :dv]
 * (reference.py:16-31). Writes out (float32, unrounded) and the natural-log
 * lse of the heads of b. Returns 2 on an allocation failure.
 */
/* Element i of a q or cache array of element type dtype, exactly. */
static double elem_to_double(const void* base, int64_t i, int dtype) {
    if (dtype == ORACLE_FP32) return (double)((const float*)base)[i];
    return half_bits_to_double(((const uint16_t*)base)[i], dtype);
}

static int attend_rows(const double* k, int64_t n, const void* q, int64_t q_sb, int64_t q_sh, int64_t b,
                       int64_t heads, int64_t dqk, int64_t dv, int dtype, double scale, float* out, float* lse) {
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
                for (int64_t c = 0; c < dqk; ++c) qd[c] = elem_to_double(q, b * q_sb + h * q_sh + c, dtype);
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
    return failed ? 2 : 0;
}

static void empty_sequence(int64_t b, int64_t heads, int64_t dv, float* out, float* lse) {
    for (int64_t h = 0; h < heads; ++h) {
        lse[b * heads + h] = -INFINITY;
        for (int64_t c = 0; c < dv; ++c) out[(b * heads + h) * dv + c] = 0.0f;
    }
}

/*
 * mla_decode_ref (reference.py:16-31), float64 throughout:
 *   s = q[b] . k^T * scale;  lse = logsumexp(s);  out = softmax(s) . k[:, :dv]
 *   n == 0  =>  out = 0, lse = -inf.
 * q is [B, H, dqk] with element strides (q_sb, q_sh, 1). out is float32
 * [B, H, dv] (not rounded: the caller rounds to the input dtype), lse is
 * float32 [B, H] natural log.
 */
int oracle_mla_decode_ref(const void* q, int64_t q_sb, int64_t q_sh, const void* kv,
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
            empty_sequence(b, heads, dv, out, lse);
            continue;
        }
        double* k = (double*)malloc((size_t)(n * dqk) * sizeof(double));
        if (!k) return 2;
#pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < n; ++t) {
            const int64_t row = token_offset(b, t, bt, bt_s0, paged, page_size, kv_s0, kv_s1);
            for (int64_t c = 0; c < dqk; ++c) k[t * dqk + c] = elem_to_double(kv, row + c, dtype);
        }
        const int rc = attend_rows(k, n, q, q_sb, q_sh, b, heads, dqk, dv, dtype, scale, out, lse);
        free(k);
        if (rc) return rc;
    }
    return 0;
}

/*
 * OCP FP8 E4M3 (the "e4m3fn" encoding: bias 7, no infinities, NaN =
 * S.1111.111) to double, exact: exponent field 0 holds the subnormals
 * m * 2^-9, field e > 0 the normals (1 + m/8) * 2^(e-7).
 */
double oracle_e4m3_to_double(uint8_t code) {
    const int sign = code >> 7, e = (code >> 3) & 15, m = code & 7;
    if (e == 15 && m == 7) return NAN;
    const double v = e == 0 ? ldexp((double)m, -9) : ldexp((double)(8 + m), e - 10);
    return sign ? -v : v;
}

/*
 * Nearest E4M3 code to x, ties to the even code (mantissa bit 0 clear).
 * Magnitudes above the midpoint 464 between the largest finite value (448)
 * and the next step (480, which is the NaN pattern) give NaN, as does NaN;
 * the sign of zero is kept. Brute force over the 127 finite magnitudes.
 */
uint8_t oracle_double_to_e4m3(double x) {
    if (isnan(x)) return 0x7f;
    const uint8_t sign = signbit(x) ? 0x80 : 0x00;
    const double a = fabs(x);
    if (a > 464.0) return (uint8_t)(sign | 0x7f);
    int best = 0;
    double best_d = INFINITY;
    for (int c = 0; c < 127; ++c) {
        const double d = fabs(oracle_e4m3_to_double((uint8_t)c) - a);
        if (d < best_d || (d == best_d && (c & 1) == 0)) {
            best_d = d;
            best = c;
        }
    }
    return (uint8_t)(sign | best);
}

void oracle_e4m3_encode(const double* in, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_double_to_e4m3(in[i]);
}

/*
 * mla_decode_ref over an fp8 cache: kv8 holds E4M3 codes, [num_blocks,
 * page_size, dqk] with element strides (kv_s0, kv_s1, 1) when paged, else
 * [batch, capacity, dqk]; row t of sequence b is dequantised as
 * e4m3(code) * kv_scale[page * sc_s0 + (t % page_size) * sc_s1] (dense:
 * kv_scale[b * sc_s0 + t * sc_s1]). q (16-bit, dtype) and the outputs are as
 * for oracle_mla_decode_ref.
 */
int oracle_mla_decode_fp8_ref(const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint8_t* kv8, int64_t kv_s0,
                              int64_t kv_s1, const float* kv_scale, int64_t sc_s0, int64_t sc_s1, const int32_t* bt,
                              int64_t bt_s0, int paged, int64_t page_size, const int32_t* seqlens, int64_t batch,
                              int64_t heads, int64_t dqk, int64_t dv, int dtype, double scale, int nthreads,
                              float* out, float* lse) {
    if (dv > dqk || dqk <= 0 || heads < 0 || batch < 0) return 1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    double table[256];
    for (int c = 0; c < 256; ++c) table[c] = oracle_e4m3_to_double((uint8_t)c);
    for (int64_t b = 0; b < batch; ++b) {
        const int64_t n = seqlens[b];
        if (n <= 0) {
            empty_sequence(b, heads, dv, out, lse);
            continue;
        }
        double* k = (double*)malloc((size_t)(n * dqk) * sizeof(double));
        if (!k) return 2;
#pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < n; ++t) {
            int64_t sidx;
            if (paged)
                sidx = (int64_t)bt[b * bt_s0 + t / page_size] * sc_s0 + (t % page_size) * sc_s1;
            else
                sidx = b * sc_s0 + t * sc_s1;
            const double sc = (double)kv_scale[sidx];
            const uint8_t* row = kv8 + token_offset(b, t, bt, bt_s0, paged, page_size, kv_s0, kv_s1);
            for (int64_t c = 0; c < dqk; ++c) k[t * dqk + c] = table[row[c]] * sc;
        }
        const int rc = attend_rows(k, n, q, q_sb, q_sh, b, heads, dqk, dv, dtype, scale, out, lse);
        free(k);
        if (rc) return rc;
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
