/*
 * iq_oracle.c -- CPU restatement of InQuant's packed-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library and the "port" CPU baseline that bench.py times beside the GPU.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product path (the inquant package and libinquant_hip.so)
 * never links, imports or calls anything here.
 *
 * Every routine restates the reference algorithm it cites (paths are into
 * the reference checkout, src/inquant/... and extensions/vllm/...).
 * Arithmetic is IEEE binary32/binary64 with round-to-nearest-even; the
 * Makefile builds with -ffp-contract=off so that no multiply-add is fused
 * where the reference rounds twice.
 *
 * Reduction order (pinned black-box against torch's CPU kernels):
 *   sum over rows      : torch CPU cascade sum (4 accumulator levels,
 *                        16-row chunks), in fp32;  mean = fl(sum / n).
 *   var_mean(corr=0)   : sequential Welford recurrence in fp64, then the
 *                        mean and m2/n are each rounded to fp32.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

#define IQO_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* scalar format helpers                                               */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* float -> bfloat16 bits, round to nearest even (torch .to(bfloat16)). */
IQO_EXPORT uint16_t iqo_f32_to_bf16(float f)
{
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

IQO_EXPORT float iqo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* float -> IEEE half bits, round to nearest even (torch .to(float16)). */
IQO_EXPORT uint16_t iqo_f32_to_f16(float f)
{
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);           /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* >= 65520 -> inf */
    if (a < 0x38800000u) {                                            /* subnormal half */
        /* value = a as float; half subnormal unit = 2^-24 */
        float v = u2f(a);
        float scaled = v * 16777216.0f;            /* exact: power of two */
        float r = rintf(scaled);                   /* RNE to integer units of 2^-24 */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t exp = ((a >> 23) - 127 + 15);
    uint32_t mant = a & 0x7fffffu;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;   /* carry may bump exponent */
    return (uint16_t)(sign | h);
}

IQO_EXPORT float iqo_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    if (exp == 0) {
        float v = (float)mant * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (mant << 13));
    return u2f(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

/* Round a float to the value representable in a 16-bit dtype (0 = f32). */
static inline float round_to(float v, int dtype)
{
    if (dtype == 1) return iqo_bf16_to_f32(iqo_f32_to_bf16(v));
    if (dtype == 2) return iqo_f16_to_f32(iqo_f32_to_f16(v));
    return v;
}

/* ------------------------------------------------------------------ */
/* torch CPU reduction orders                                          */
/* ------------------------------------------------------------------ */

static int ceil_log2_i64(int64_t x)
{
    int r = 0;
    if (x <= 1) return 0;
    x -= 1;
    while (x) { ++r; x >>= 1; }
    return r;
}

/*
 * Sum of n fp32 values v[0], v[stride], ... in torch's CPU cascade order
 * (the accumulator levels of aten's multi_row_sum, used by
 * codec.py:205-206 `samples.abs().mean(-2)` / `samples.mean(-2)`).
 */
static float cascade_sum(const float *v, int64_t n, int64_t stride, int use_abs)
{
    const int levels = 4;
    int lp = ceil_log2_i64(n) / levels;
    if (lp < 4) lp = 4;
    const int64_t step = (int64_t)1 << lp;
    const int64_t mask = step - 1;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int64_t i = 0;
    while (i + step <= n) {
        for (int64_t j = 0; j < step; ++j, ++i) {
            float x = v[i * stride];
            acc[0] = acc[0] + (use_abs ? fabsf(x) : x);
        }
        for (int j = 1; j < levels; ++j) {
            acc[j] = acc[j] + acc[j - 1];
            acc[j - 1] = 0.0f;
            if ((i & (mask << (j * lp))) != 0) break;
        }
    }
    for (; i < n; ++i) {
        float x = v[i * stride];
        acc[0] = acc[0] + (use_abs ? fabsf(x) : x);
    }
    for (int j = 1; j < levels; ++j) acc[0] = acc[0] + acc[j];
    return acc[0];
}

/*
 * torch CPU "row_sum": the n values are read as an [n/4, 4] array, each of
 * the 4 interleaved lanes is cascade-summed, the n % 4 leftovers are added
 * to lane 0, then lanes 1..3 are added to lane 0 in order.
 */
static float ilp4_sum(const float *v, int64_t n, int64_t stride, int use_abs)
{
    int64_t g = n / 4;
    float part[4];
    for (int k = 0; k < 4; ++k) part[k] = cascade_sum(v + k * stride, g, 4 * stride, use_abs);
    for (int64_t i = 4 * g; i < n; ++i) {
        float x = v[i * stride];
        part[0] = part[0] + (use_abs ? fabsf(x) : x);
    }
    return ((part[0] + part[1]) + part[2]) + part[3];
}

/*
 * Column sum over n rows in the order torch's CPU outer reduction uses for
 * a [n, D] input with contiguous columns: columns [0, 32*floor(D/32)) are
 * cascade-summed four 8-wide vectors at a time; the remaining columns use
 * row_sum.  Inputs narrower than 8 columns take the scalar path: columns in
 * groups of 4 are cascade-summed, the rest use row_sum.
 */
IQO_EXPORT int64_t iqo_cascade_columns(int64_t D)
{
    const int64_t W = 8;
    return D >= W ? (D / (4 * W)) * (4 * W) : (D / 4) * 4;
}

static float column_sum(const float *v, int64_t n, int64_t stride, int64_t c, int64_t D, int use_abs)
{
    return c < iqo_cascade_columns(D) ? cascade_sum(v, n, stride, use_abs) : ilp4_sum(v, n, stride, use_abs);
}

/*
 * Per-channel statistics of one [T, D] row (codec.py:200-210):
 * sampled saliency mean(|x|) and sampled mean over rows 0, s, 2s, ...;
 * for min_error, the full-row var_mean (Welford, fp64) and
 * err = var + (mean - sampled_mean)^2 in fp32; amax |x| over all rows.
 */
IQO_EXPORT void iqo_k4_stats(const float *x, int64_t T, int64_t D, int64_t stride,
                             int min_error, float *sal, float *smean, float *err, float *amax)
{
    int64_t ns = (T + stride - 1) / stride;
    for (int64_t c = 0; c < D; ++c) {
        float sa = column_sum(x + c, ns, stride * D, c, D, 1);
        float sm = column_sum(x + c, ns, stride * D, c, D, 0);
        sal[c] = sa / (float)ns;
        smean[c] = sm / (float)ns;
        float mx = 0.0f;
        for (int64_t t = 0; t < T; ++t) {
            float a = fabsf(x[t * D + c]);
            if (a > mx) mx = a;
        }
        amax[c] = mx;
        if (min_error && err) {
            double mean = 0.0, m2 = 0.0;
            for (int64_t t = 0; t < T; ++t) {
                double val = (double)x[t * D + c];
                double nf = (double)(t + 1);
                double delta = val - mean;
                mean = mean + delta / nf;
                double nd = val - mean;
                m2 = m2 + delta * nd;
            }
            float var = (float)(m2 / (double)T);
            float fmean = (float)mean;
            float diff = fmean - smean[c];
            float sq = diff * diff;
            err[c] = var + sq;
        }
    }
}

/* ------------------------------------------------------------------ */
/* donor selection (codec.py:137-178)                                  */
/* ------------------------------------------------------------------ */

static inline int gt_nan_high(float a, float b) { return a > b || (isnan(a) && !isnan(b)); }
static inline int lt_nan_high(float a, float b) { return a < b || (!isnan(a) && isnan(b)); }
static inline int eq_nan(float a, float b) { return a == b || (isnan(a) && isnan(b)); }

/*
 * One row of _reuse_map: stable top-`count` by saliency (ties to the lower
 * channel), sorted ascending; optional min_error pool; then `count`
 * sequential donor picks (immediate neighbours first, else the channels
 * nearest either boundary of the source's contiguous salient run), each the
 * first-index argmin of saliency among the candidates.
 */
IQO_EXPORT void iqo_reuse_map_row(const float *sal, const float *err, int64_t D, int64_t count,
                                  int64_t *src, int64_t *don, uint8_t *work /* 2*D bytes */)
{
    uint8_t *selected = work, *available = work + D;
    for (int64_t c = 0; c < D; ++c) {
        int64_t rank = 0;
        for (int64_t o = 0; o < D; ++o)
            if (gt_nan_high(sal[o], sal[c]) || (eq_nan(sal[o], sal[c]) && o < c)) ++rank;
        selected[c] = (uint8_t)(rank < count);
    }
    int64_t k = 0;
    for (int64_t c = 0; c < D; ++c)
        if (selected[c]) src[k++] = c;
    if (err) {
        for (int64_t c = 0; c < D; ++c) {
            float ec = selected[c] ? INFINITY : err[c];
            int64_t rank = 0;
            for (int64_t o = 0; o < D; ++o) {
                float eo = selected[o] ? INFINITY : err[o];
                if (lt_nan_high(eo, ec) || (eq_nan(eo, ec) && o < c)) ++rank;
            }
            available[c] = (uint8_t)(rank < count);
        }
    } else {
        for (int64_t c = 0; c < D; ++c) available[c] = (uint8_t)!selected[c];
    }
    for (int64_t i = 0; i < count; ++i) {
        int64_t s = src[i];
        int any_imm = (s - 1 >= 0 && available[s - 1]) || (s + 1 < D && available[s + 1]);
        int64_t best = -1;
        float bestv = INFINITY;
        if (any_imm) {
            for (int64_t p = 0; p < D; ++p) {
                float v = (available[p] && (p == s - 1 || p == s + 1)) ? sal[p] : INFINITY;
                if (best < 0 || lt_nan_high(v, bestv)) { best = p; bestv = v; }
            }
        } else {
            int64_t left = -1, right = D;
            for (int64_t p = 0; p < s; ++p) if (!selected[p]) left = p;
            for (int64_t p = D - 1; p > s; --p) if (!selected[p]) right = p;
            left += 1;
            right -= 1;
            int64_t nearest = D + 1;
            for (int64_t p = 0; p < D; ++p) {
                if (!available[p]) continue;
                int64_t dl = llabs(p - left), dr = llabs(p - right);
                int64_t d = dl < dr ? dl : dr;
                if (d < nearest) nearest = d;
            }
            for (int64_t p = 0; p < D; ++p) {
                int64_t dl = llabs(p - left), dr = llabs(p - right);
                int64_t d = dl < dr ? dl : dr;
                float v = (available[p] && d == nearest) ? sal[p] : INFINITY;
                if (best < 0 || lt_nan_high(v, bestv)) { best = p; bestv = v; }
            }
        }
        don[i] = best;
        available[best] = 0;
    }
}

/* OpenMP thread count of the oracle's parallel loops (CPU-baseline timing). */
IQO_EXPORT void iqo_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

IQO_EXPORT void iqo_reuse_map(const float *sal, const float *err, int64_t rows, int64_t D,
                              int64_t count, int64_t *src, int64_t *don)
{
    #pragma omp parallel
    {
        uint8_t *work = (uint8_t *)malloc((size_t)(2 * D));
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r)
            iqo_reuse_map_row(sal + r * D, err ? err + r * D : NULL, D, count,
                              src + r * count, don + r * count, work);
        free(work);
    }
}

/* ------------------------------------------------------------------ */
/* K4 quantize / dequantize (codec.py:181-243, codec.py:112-134)       */
/* ------------------------------------------------------------------ */

/*
 * x: fp32 [rows, T, D] contiguous (rows = batch*heads).  Outputs per row:
 * payload [T, D/2], scales [D], src/don [count] (int64), padding [count].
 * Returns 0, or -1 if x holds a non-finite value (codec.py:197).
 */
IQO_EXPORT int iqo_k4_quantize(const float *x, int64_t rows, int64_t T, int64_t D, int64_t count,
                               int64_t stride, int min_error, uint8_t *payload, float *scales,
                               int64_t *src, int64_t *don, float *padding)
{
    int64_t n = rows * T * D;
    for (int64_t i = 0; i < n; ++i)
        if (!isfinite(x[i])) return -1;
    #pragma omp parallel
    {
        float *sal = (float *)malloc(sizeof(float) * (size_t)D * 4);
        float *smean = sal + D, *err = sal + 2 * D, *amax = sal + 3 * D;
        uint8_t *work = (uint8_t *)malloc((size_t)(3 * D));
        uint8_t *slots = (uint8_t *)malloc((size_t)D);
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            const float *xr = x + r * T * D;
            int64_t *sr = src + r * count, *dr = don + r * count;
            iqo_k4_stats(xr, T, D, stride, min_error, sal, smean, err, amax);
            iqo_reuse_map_row(sal, min_error ? err : NULL, D, count, sr, dr, work);
            uint8_t *sel = work + 2 * D;
            memset(sel, 0, (size_t)D);
            for (int64_t i = 0; i < count; ++i) sel[sr[i]] = 1;
            float *sc = scales + r * D;
            for (int64_t c = 0; c < D; ++c) {
                float s = amax[c] / (sel[c] ? 127.0f : 7.0f);
                sc[c] = s < FLT_MIN ? FLT_MIN : s;
            }
            for (int64_t t = 0; t < T; ++t) {
                const float *xt = xr + t * D;
                for (int64_t c = 0; c < D; ++c) {
                    float q = rintf(xt[c] / sc[c]);
                    q = q < -7.0f ? -7.0f : (q > 7.0f ? 7.0f : q);
                    slots[c] = (uint8_t)(q + 8.0f);
                }
                for (int64_t i = 0; i < count; ++i) {
                    float q = rintf(xt[sr[i]] / sc[sr[i]]);
                    q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
                    uint8_t code = (uint8_t)(q + 128.0f);
                    slots[sr[i]] = (uint8_t)(code >> 4);
                    slots[dr[i]] = (uint8_t)(code & 15);
                }
                uint8_t *pt = payload + (r * T + t) * (D / 2);
                for (int64_t j = 0; j < D / 2; ++j)
                    pt[j] = (uint8_t)(slots[2 * j] | (slots[2 * j + 1] << 4));
            }
            for (int64_t i = 0; i < count; ++i) padding[r * count + i] = smean[dr[i]];
        }
        free(sal);
        free(work);
        free(slots);
    }
    return 0;
}

/* Dequantize one K4 tensor to fp32, then round to `dtype` (0 f32, 1 bf16, 2 f16). */
IQO_EXPORT void iqo_k4_dequantize(const uint8_t *payload, const float *scales, const int64_t *src,
                                  const int64_t *don, const float *padding, int64_t rows, int64_t T,
                                  int64_t D, int64_t count, int dtype, float *out)
{
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float *sc = scales + r * D;
        for (int64_t t = 0; t < T; ++t) {
            const uint8_t *pt = payload + (r * T + t) * (D / 2);
            float *o = out + (r * T + t) * D;
            for (int64_t c = 0; c < D; ++c) {
                int slot = (c & 1) ? (pt[c >> 1] >> 4) : (pt[c >> 1] & 15);
                o[c] = ((float)slot - 8.0f) * sc[c];
            }
            for (int64_t i = 0; i < count; ++i) {
                int64_t s = src[r * count + i], d = don[r * count + i];
                int hi = (s & 1) ? (pt[s >> 1] >> 4) : (pt[s >> 1] & 15);
                int lo = (d & 1) ? (pt[d >> 1] >> 4) : (pt[d >> 1] & 15);
                o[s] = ((float)((hi << 4) | lo) - 128.0f) * sc[s];
            }
            for (int64_t i = 0; i < count; ++i) o[don[r * count + i]] = padding[r * count + i];
            for (int64_t c = 0; c < D; ++c) o[c] = round_to(o[c], dtype);
        }
    }
}

/* ------------------------------------------------------------------ */
/* V2/V4 group-wise values (value_codec.py:51-72, value_codec.py:38-48) */
/* ------------------------------------------------------------------ */

/*
 * x: fp32 [rows, D] (rows = batch*heads*tokens).  Outputs payload
 * [rows, D*bits/8], f16 bits scales/offsets [rows, D/group].
 * Returns 0, or -1 if a value or a stored f16 parameter is non-finite.
 */
IQO_EXPORT int iqo_v_quantize(const float *x, int64_t rows, int64_t D, int bits, int group,
                              uint8_t *payload, uint16_t *scales, uint16_t *offsets)
{
    int bad = 0;
    const int levels = (1 << bits) - 1;
    const int per_byte = 8 / bits;
    #pragma omp parallel for schedule(static) reduction(|:bad)
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * D;
        uint8_t *pr = payload + r * (D / per_byte);
        memset(pr, 0, (size_t)(D / per_byte));
        for (int64_t g = 0; g < D / group; ++g) {
            const float *xg = xr + g * group;
            float lo = xg[0], hi = xg[0];
            for (int j = 0; j < group; ++j) {
                if (!isfinite(xg[j])) bad = 1;
                if (xg[j] < lo) lo = xg[j];
                if (xg[j] > hi) hi = xg[j];
            }
            uint16_t off = iqo_f32_to_f16(lo);
            float s = (hi - lo) / (float)levels;
            const float tiny = 6.103515625e-05f;
            if (s < tiny) s = tiny;
            uint16_t sch = iqo_f32_to_f16(s);
            offsets[r * (D / group) + g] = off;
            scales[r * (D / group) + g] = sch;
            float offf = iqo_f16_to_f32(off), scf = iqo_f16_to_f32(sch);
            if (!isfinite(offf) || !isfinite(scf)) bad = 1;
            for (int j = 0; j < group; ++j) {
                float q = rintf((xg[j] - offf) / scf);
                q = q < 0.0f ? 0.0f : (q > (float)levels ? (float)levels : q);
                int64_t ch = g * group + j;
                uint8_t code = (uint8_t)q;
                pr[ch / per_byte] |= (uint8_t)(code << ((ch % per_byte) * bits));
            }
        }
    }
    return bad ? -1 : 0;
}

IQO_EXPORT void iqo_v_dequantize(const uint8_t *payload, const uint16_t *scales, const uint16_t *offsets,
                                 int64_t rows, int64_t D, int bits, int group, int dtype, float *out)
{
    const int per_byte = 8 / bits;
    const int mask = (1 << bits) - 1;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < D; ++c) {
            int code = (payload[r * (D / per_byte) + c / per_byte] >> ((c % per_byte) * bits)) & mask;
            float sc = iqo_f16_to_f32(scales[r * (D / group) + c / group]);
            float of = iqo_f16_to_f32(offsets[r * (D / group) + c / group]);
            float prod = (float)code * sc;
            out[r * D + c] = round_to(prod + of, dtype);
        }
    }
}

/* ------------------------------------------------------------------ */
/* role maps (triton_attention.py:301-309; layout.py:73-77)            */
/* ------------------------------------------------------------------ */

/* out: [heads, D] int16 roles: -1 normal, donor index for a source, -2-i for donor i. */
IQO_EXPORT void iqo_role_map(const int64_t *src, const int64_t *don, int64_t heads, int64_t D,
                             int64_t count, int16_t *out)
{
    for (int64_t h = 0; h < heads; ++h) {
        for (int64_t c = 0; c < D; ++c) out[h * D + c] = -1;
        for (int64_t i = 0; i < count; ++i) out[h * D + src[h * count + i]] = (int16_t)don[h * count + i];
        for (int64_t i = 0; i < count; ++i) out[h * D + don[h * count + i]] = (int16_t)(-2 - i);
    }
}

/* ------------------------------------------------------------------ */
/* attention over materialized K/V (qwen_fused.py:21-30)               */
/* ------------------------------------------------------------------ */

/*
 * Single-query GQA attention in fp64 over K/V already rounded to the query
 * dtype: q [Hq, D], k/v [H, T, D] (fp32 holding exact dtype values),
 * out [Hq, D] fp64.  Query head h reads KV head h / (Hq / H).
 */
IQO_EXPORT void iqo_attend(const float *q, const float *k, const float *v, int64_t Hq, int64_t H,
                           int64_t T, int64_t D, double scale, double *out)
{
    const int64_t G = Hq / H;
    #pragma omp parallel
    {
        double *s = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
        #pragma omp for schedule(static)
        for (int64_t h = 0; h < Hq; ++h) {
            const int64_t kv = h / G;
            const float *qh = q + h * D;
            double m = -INFINITY;
            for (int64_t t = 0; t < T; ++t) {
                const float *kt = k + (kv * T + t) * D;
                double acc = 0.0;
                for (int64_t d = 0; d < D; ++d) acc += (double)qh[d] * (double)kt[d];
                s[t] = acc * scale;
                if (s[t] > m) m = s[t];
            }
            double l = 0.0;
            double *o = out + h * D;
            for (int64_t d = 0; d < D; ++d) o[d] = 0.0;
            for (int64_t t = 0; t < T; ++t) {
                double p = exp(s[t] - m);
                l += p;
                const float *vt = v + (kv * T + t) * D;
                for (int64_t d = 0; d < D; ++d) o[d] += p * (double)vt[d];
            }
            for (int64_t d = 0; d < D; ++d) o[d] /= l;
        }
        free(s);
    }
}

/*
 * Test support for the GPU tile encoder, not part of the reference's
 * algorithm: the Welford step's delta / n is computed on the GPU as
 *   q0 = delta * RN(1/n);  r = fma(-q0, n, delta);  q = fma(r, RN(1/n), q0)
 * which must equal the IEEE quotient for every n <= n_max.  Checks
 * `samples` deltas per n drawn as differences of random floats and a
 * running double mean (the operands the recurrence produces); returns the
 * number of mismatches.
 */
int64_t iqo_check_recip_division(int64_t n_max, int64_t samples, uint64_t seed)
{
    int64_t bad = 0;
    uint64_t s = seed;
    for (int64_t n = 1; n <= n_max; ++n) {
        const double nd = (double)n, y = 1.0 / nd;
        for (int64_t i = 0; i < samples; ++i) {
            s += 0x9E3779B97F4A7C15ull;
            uint64_t z = s;
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
            z ^= z >> 31;
            /* a float of random sign, exponent in [-40, 40) and mantissa, minus a double "mean" */
            uint32_t fb = (uint32_t)(z & 0x807fffffu) | ((uint32_t)(87 + ((z >> 32) % 80)) << 23);
            float xf;
            memcpy(&xf, &fb, 4);
            double mean = (double)(int64_t)(z >> 40) * 0x1p-20 * ((z >> 39) & 1 ? 1.0 : 1e-9);
            const double delta = (double)xf - mean;
            const double q0 = delta * y;
            const double r = fma(-q0, nd, delta);
            const double q = fma(r, y, q0);
            const double ref = delta / nd;
            if (memcmp(&q, &ref, 8) != 0) ++bad;
        }
    }
    return bad;
}
