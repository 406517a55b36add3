// K4 neighbor-slot encoder and standalone donor selector (gfx950).
//
// One 256-thread workgroup encodes one (batch, head) row of x[B, H, T, D]:
//   phase 1  per-channel statistics: sampled saliency and mean in torch's
//            CPU summation order, full-block amax, and for min_error the
//            fp64 Welford var_mean (codec.py:200-210);
//   phase 2  donor selection by wavefront 0 (select_dev.h);
//   phase 3  scales, 4-bit slots, 8-bit salient codes split across the
//            source and donor slots, nibble packing, padding (codec.py:218-233).
// Results are bit-identical to the reference CPU implementation.
#include "select_dev.h"
#include "v_rows_dev.h"

#include <cstdarg>
#include <cstdio>

namespace {

constexpr int K4_THREADS = 256;

struct K4Args {
    const void *x;
    int dt;
    int64_t sb, sh, st, sc;   // element strides
    int64_t H, T, D, count, stride;
    int min_error;
    uint8_t *payload;
    float *scales;
    void *src, *don;
    int desc_bytes;
    float *padding;
    int *bad;
    // page mode (k4_encode_tile<..., true>): row (b, h) is written into the
    // physical page ids[b] of `pool` (byte offsets of the page fields), with
    // an int16 role map instead of descriptors, and the value rows of v
    // (element strides vsb, vsh, vst) are V2-encoded into the same page
    uint8_t *pool;
    int64_t pool_pages, page_bytes;
    const void *ids;
    int id_bytes;
    int64_t off_kpay, off_kscale, off_kmap, off_kpad, off_vpay, off_vscale, off_voff;
    const uint16_t *v;
    int64_t vsb, vsh, vst;
    int *vbad, *badid, *clear;  // value flag; out-of-range page id flag; flag triple the next page launch uses, zeroed here
    // page mode, optional: page b starts at token row page_rows[b] of x / v
    // (offsets page_rows[b] * st, page_rows[b] * vst) instead of b * sb, b * vsb
    const int64_t *page_rows;
    // fused key/value mode (k4_encode_tile<..., VB = 2 or 4>): the value rows
    // of v are encoded group-wise into the outputs of iq_v_quantize
    uint8_t *vpayload;
    uint16_t *vscales, *voffsets;
    // k4_encode_kernel with long rows: statistics, selection, scales and
    // descriptors only; k4_quantize_generic then writes the payload
    int split;
};

__device__ __forceinline__ void store_desc(void *p, int64_t i, int v, int bytes)
{
    if (bytes == 1) ((uint8_t *)p)[i] = (uint8_t)v;
    else if (bytes == 4) ((int32_t *)p)[i] = v;
    else ((int64_t *)p)[i] = v;
}

// Sampled sums of one channel in torch's order (cascade, or interleaved row_sum).
// Calls f(v, i) for i = 0 .. n - 1 in order with v the element at
// base + (i * mul + add) * step, loading SEQ_PF elements ahead of their use
// (one memory round trip per SEQ_PF elements of a sequential reduction).
constexpr int SEQ_PF = 16;

template <int DT, typename F>
__device__ __forceinline__ void for_each_seq_t(const void *x, int64_t base, int64_t step, int64_t n, int64_t mul,
                                               int64_t add, F &f)
{
    // whole groups without a bound check per element, the next group's loads
    // issued before the current group is reduced (its round trip overlaps
    // SEQ_PF steps of the reduction), then the ragged end
    const int64_t nfull = n - n % SEQ_PF;
    float cur[SEQ_PF];
    if (nfull > 0) {
#pragma unroll
        for (int u = 0; u < SEQ_PF; ++u)
            cur[u] = iq_load_f32(x, base + (u * mul + add) * step, DT);   // DT constant: no branch per load
    }
    for (int64_t i0 = 0; i0 < nfull; i0 += SEQ_PF) {
        float nxt[SEQ_PF];
        const int64_t i1 = i0 + SEQ_PF < nfull ? i0 + SEQ_PF : i0;   // the last group reloads itself
#pragma unroll
        for (int u = 0; u < SEQ_PF; ++u)
            nxt[u] = iq_load_f32(x, base + ((i1 + u) * mul + add) * step, DT);
#pragma unroll
        for (int u = 0; u < SEQ_PF; ++u) f(cur[u], i0 + u);
#pragma unroll
        for (int u = 0; u < SEQ_PF; ++u) cur[u] = nxt[u];
    }
    if (nfull < n) {
        float v[SEQ_PF];
#pragma unroll
        for (int u = 0; u < SEQ_PF; ++u) {
            const int64_t i = nfull + u < n ? nfull + u : n - 1;
            v[u] = iq_load_f32(x, base + (i * mul + add) * step, DT);
        }
#pragma unroll
        for (int u = 0; u < SEQ_PF; ++u)
            if (nfull + u < n) f(v[u], nfull + u);
    }
}

// RN(1 / n) for an integer 1 <= n <= 2^24: the float reciprocal (exact
// input, within a few ulp) and two Newton steps with fma.  After them the
// relative error before the last rounding is ~2^-84, while 1 / n lies at
// least 2^-78 (relative) from a rounding midpoint of the doubles for
// n <= 2^24, so the result is the correctly rounded reciprocal
// (tests/test_welford_division.py checks every such n with the float start
// off by up to 4 ulp either way).
__device__ __forceinline__ double iq_rcp_small_int(uint32_t n)
{
    const double d = (double)n;
    double y = (double)__builtin_amdgcn_rcpf((float)n);
    y = __builtin_fma(y, __builtin_fma(-d, y, 1.0), y);
    return __builtin_fma(y, __builtin_fma(-d, y, 1.0), y);
}

// lane l's double, read by the whole wave (l uniform)
__device__ __forceinline__ double iq_read_lane_f64(double v, int l)
{
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

template <typename F>
__device__ __forceinline__ void for_each_seq(const void *x, int dt, int64_t base, int64_t step, int64_t n, int64_t mul,
                                             int64_t add, F &&f)
{
    switch (dt) {
    case IQ_BF16: for_each_seq_t<IQ_BF16>(x, base, step, n, mul, add, f); break;
    case IQ_F16: for_each_seq_t<IQ_F16>(x, base, step, n, mul, add, f); break;
    case IQ_F64: for_each_seq_t<IQ_F64>(x, base, step, n, mul, add, f); break;
    default: for_each_seq_t<IQ_F32>(x, base, step, n, mul, add, f); break;
    }
}

__device__ __forceinline__ void sampled_sums(const void *x, int dt, int64_t base, int64_t step, int64_t ns, bool cascade_col,
                             float &sum_abs, float &sum)
{
    if (cascade_col) {
        IqCascade a, s;
        a.init(ns);
        s.init(ns);
        for_each_seq(x, dt, base, step, ns, 1, 0, [&](float v, int64_t) {
            a.add(fabsf(v));
            s.add(v);
        });
        sum_abs = a.finish();
        sum = s.finish();
    } else {
        const int64_t g = ns / 4;
        float pa[4], ps[4];
        for (int k = 0; k < 4; ++k) {
            IqCascade a, s;
            a.init(g);
            s.init(g);
            for_each_seq(x, dt, base, step, g, 4, k, [&](float v, int64_t) {
                a.add(fabsf(v));
                s.add(v);
            });
            pa[k] = a.finish();
            ps[k] = s.finish();
        }
        for (int64_t r = 4 * g; r < ns; ++r) {
            const float v = iq_load_f32(x, base + r * step, dt);
            pa[0] = __fadd_rn(pa[0], fabsf(v));
            ps[0] = __fadd_rn(ps[0], v);
        }
        sum_abs = __fadd_rn(__fadd_rn(__fadd_rn(pa[0], pa[1]), pa[2]), pa[3]);
        sum = __fadd_rn(__fadd_rn(__fadd_rn(ps[0], ps[1]), ps[2]), ps[3]);
    }
}

__global__ __launch_bounds__(K4_THREADS) void k4_encode_kernel(K4Args a)
{
    __shared__ float s_sal[IQ_MAXD];
    __shared__ float s_smean[IQ_MAXD];
    __shared__ float s_err[IQ_MAXD];
    __shared__ float s_scale[IQ_MAXD];
    __shared__ int16_t s_src_of[IQ_MAXD];
    __shared__ uint8_t s_is_src[IQ_MAXD];
    __shared__ int16_t s_src[IQ_MAXD / 2];
    __shared__ int16_t s_don[IQ_MAXD / 2];
    __shared__ int s_bad;

    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t b = row / a.H, h = row % a.H;
    const int64_t base = b * a.sb + h * a.sh;
    const int64_t T = a.T, D = a.D;
    const int64_t ns = (T + a.stride - 1) / a.stride;
    const int64_t ncasc = iq_cascade_columns(D);

    if (tid == 0) s_bad = 0;
    __syncthreads();

    // ---- phase 1: per-channel statistics (one thread per channel).  Every
    // lane of a wave that has channels left runs the loop (lanes past D repeat
    // channel D - 1 and write nothing), so the reciprocals that lanes compute
    // for each other below are always there to read.
    const int lane = tid & 63;
    for (int64_t c0 = tid - lane; c0 < D; c0 += K4_THREADS) {
        const bool own = c0 + lane < D;
        const int64_t c = own ? c0 + lane : D - 1;
        const int64_t cb = base + c * a.sc;
        float sum_abs, sum;
        sampled_sums(a.x, a.dt, cb, a.st * a.stride, ns, c < ncasc, sum_abs, sum);
        const float smean = sum / (float)ns;
        if (own) {
            s_sal[c] = sum_abs / (float)ns;
            s_smean[c] = smean;
        }
        float amax = 0.0f;
        bool bad = false;
        double mean = 0.0, m2 = 0.0, ygrp = 0.0;
        const bool me = a.min_error;
        // rows of up to 2^24 tokens take the reciprocal from iq_rcp_small_int
        auto stats = [&](auto small) {
            for_each_seq(a.x, a.dt, cb, a.st, T, 1, 0, [&](float v, int64_t t) {
            bad |= !iq_isfinite(v);
            amax = fmaxf(amax, fabsf(v));
            if (me) {
                // delta / n as RN(1 / n) (off the dependent chain) and one
                // remainder correction: the correctly rounded quotient
                // (tests/test_welford_division.py, n up to 2^24)
                const double n = decltype(small)::value ? (double)(uint32_t)(t + 1) : (double)(t + 1);
                // rows of up to 2^24 tokens: at the start of each group of
                // SEQ_PF steps (t a multiple of SEQ_PF there, for_each_seq_t's
                // groups) lane l computes RN(1 / (t + 1 + l % SEQ_PF)), and
                // step t reads it from lane t % SEQ_PF: one reciprocal per
                // group instead of one per step
                double y;
                if constexpr (decltype(small)::value) {
                    if ((t & (SEQ_PF - 1)) == 0) ygrp = iq_rcp_small_int((uint32_t)(t + 1 + (lane & (SEQ_PF - 1))));
                    y = iq_read_lane_f64(ygrp, (int)(t & (SEQ_PF - 1)));
                } else {
                    y = 1.0 / n;
                }
                const double dv = (double)v;
                const double delta = __dsub_rn(dv, mean);
                const double q0 = __dmul_rn(delta, y);
                const double r = __builtin_fma(-q0, n, delta);
                mean = __dadd_rn(mean, __builtin_fma(r, y, q0));
                const double nd = __dsub_rn(dv, mean);
                m2 = __dadd_rn(m2, __dmul_rn(delta, nd));
            }
            });
        };
        if (T <= (int64_t(1) << 24)) stats(std::true_type{});
        else stats(std::false_type{});
        if (a.min_error) {
            const float var = (float)(m2 / (double)T);
            const float diff = __fsub_rn((float)mean, smean);
            if (own) s_err[c] = __fadd_rn(var, __fmul_rn(diff, diff));
        }
        if (own) s_scale[c] = amax;
        if (bad) s_bad = 1;
    }
    __syncthreads();

    // ---- phase 2: selection by wavefront 0
    if (tid < 64) {
        iq_select_wave(s_sal, a.min_error ? s_err : nullptr, (int)D, (int)a.count, s_src, s_don, s_is_src,
                       s_src_of);
    }
    __syncthreads();

    // ---- scales and descriptors
    const float flt_min = 1.17549435e-38f;
    for (int64_t c = tid; c < D; c += K4_THREADS) {
        const float s = s_scale[c] / (s_is_src[c] ? 127.0f : 7.0f);
        const float sc = s < flt_min ? flt_min : s;
        s_scale[c] = sc;
        a.scales[row * D + c] = sc;
    }
    for (int64_t i = tid; i < a.count; i += K4_THREADS) {
        store_desc(a.src, row * a.count + i, s_src[i], a.desc_bytes);
        store_desc(a.don, row * a.count + i, s_don[i], a.desc_bytes);
        a.padding[row * a.count + i] = s_smean[s_don[i]];
    }
    if (tid == 0 && s_bad) atomicOr(a.bad, 1);
    __syncthreads();

    if (a.split) return;

    // ---- phase 3: slots and nibble packing, one payload byte per step, the
    // inputs of P3_UNROLL steps loaded before any is used
    const int64_t half = D / 2;
    uint8_t *out = a.payload + row * T * half;
    constexpr int P3_UNROLL = 8;
    for (int64_t idx0 = tid; idx0 < T * half; idx0 += (int64_t)K4_THREADS * P3_UNROLL) {
        float xv[P3_UNROLL][2];
#pragma unroll
        for (int u = 0; u < P3_UNROLL; ++u) {
            const int64_t idx = idx0 + (int64_t)u * K4_THREADS;
            const int64_t ic = idx < T * half ? idx : T * half - 1;
            const int64_t t = ic / half, j = ic - t * half;
            const int64_t tb = base + t * a.st;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int64_t c = 2 * j + e;
                const int16_t owner = s_src_of[c];
                const int64_t sc = (s_is_src[c] || owner < 0) ? c : owner;    // the channel slot c encodes
                xv[u][e] = iq_load_f32(a.x, tb + sc * a.sc, a.dt);
            }
        }
#pragma unroll
        for (int u = 0; u < P3_UNROLL; ++u) {
            const int64_t idx = idx0 + (int64_t)u * K4_THREADS;
            if (idx >= T * half) break;
            const int64_t j = idx % half;
            uint32_t slots[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int64_t c = 2 * j + e;
                const int16_t owner = s_src_of[c];
                float q;
                if (s_is_src[c] || owner >= 0) {
                    const int64_t sc = s_is_src[c] ? c : owner;
                    q = rintf(xv[u][e] / s_scale[sc]);
                    q = fminf(fmaxf(q, -127.0f), 127.0f);
                    const uint32_t code = (uint32_t)(q + 128.0f);
                    slots[e] = s_is_src[c] ? (code >> 4) : (code & 15u);
                } else {
                    q = rintf(xv[u][e] / s_scale[c]);
                    q = fminf(fmaxf(q, -7.0f), 7.0f);
                    slots[e] = (uint32_t)(q + 8.0f);
                }
            }
            out[idx] = (uint8_t)(slots[0] | (slots[1] << 4));
        }
    }
}

// Phase 3 of k4_encode_kernel for long rows, spread over the tokens: grid
// (token tiles of Q_TOKENS, rows); each workgroup takes the row's scales and
// descriptors from global memory (written by the statistics launch) and
// quantizes its tokens exactly as phase 3 does.
constexpr int64_t Q_TOKENS = 64;

__global__ __launch_bounds__(K4_THREADS) void k4_quantize_generic(K4Args a)
{
    __shared__ float s_scale[IQ_MAXD];
    __shared__ int16_t s_src_of[IQ_MAXD];
    __shared__ uint8_t s_is_src[IQ_MAXD];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.y, b = row / a.H, h = row % a.H;
    const int64_t base = b * a.sb + h * a.sh, D = a.D, half = D / 2;
    auto desc = [&](const void *p, int64_t i) -> int {
        return a.desc_bytes == 1 ? ((const uint8_t *)p)[i]
               : a.desc_bytes == 4 ? ((const int32_t *)p)[i] : (int)((const int64_t *)p)[i];
    };
    for (int64_t c = tid; c < D; c += K4_THREADS) {
        s_scale[c] = a.scales[row * D + c];
        s_is_src[c] = 0;
        s_src_of[c] = -1;
    }
    __syncthreads();
    for (int64_t i = tid; i < a.count; i += K4_THREADS) {
        const int sc = desc(a.src, row * a.count + i), dn = desc(a.don, row * a.count + i);
        s_is_src[sc] = 1;
        s_src_of[dn] = (int16_t)sc;
    }
    __syncthreads();
    const int64_t t0 = (int64_t)blockIdx.x * Q_TOKENS, t1 = t0 + Q_TOKENS < a.T ? t0 + Q_TOKENS : a.T;
    uint8_t *out = a.payload + row * a.T * half;
    for (int64_t idx = t0 * half + tid; idx < t1 * half; idx += K4_THREADS) {
        const int64_t t = idx / half, j = idx - t * half;
        const int64_t tb = base + t * a.st;
        uint32_t slots[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int64_t c = 2 * j + e;
            const int16_t owner = s_src_of[c];
            float q;
            if (s_is_src[c] || owner >= 0) {
                const int64_t sc = s_is_src[c] ? c : owner;
                q = rintf(iq_load_f32(a.x, tb + sc * a.sc, a.dt) / s_scale[sc]);
                q = fminf(fmaxf(q, -127.0f), 127.0f);
                const uint32_t code = (uint32_t)(q + 128.0f);
                slots[e] = s_is_src[c] ? (code >> 4) : (code & 15u);
            } else {
                q = rintf(iq_load_f32(a.x, tb + c * a.sc, a.dt) / s_scale[c]);
                q = fminf(fmaxf(q, -7.0f), 7.0f);
                slots[e] = (uint32_t)(q + 8.0f);
            }
        }
        out[idx] = (uint8_t)(slots[0] | (slots[1] << 4));
    }
}

// ---------------------------------------------------------------------------
// Tile encoder for the cache shapes: D = 128, 16-bit input, T <= 256 tokens,
// channel-contiguous rows.  The block streams through LDS in 32-token chunks
// (double-buffered, 16-byte loads, three chunks in flight while the current
// one is consumed), twice:
//   pass 1  waves 0-1: the fp64 Welford var_mean of channel tid (min_error
//           only); delta / n uses a table of RN(1/n) and one remainder fma,
//           which is the correctly rounded quotient for n <= 256 (sealed
//           blocks: one fma with compile-time constants, see step_c);
//           waves 2-3: sampled sums (torch cascade order), amax and
//           finiteness as an integer max of the 16-bit magnitudes;
//   then    donor selection by the whole workgroup (iq_select_tile128);
//           the sequential donor picks run on one wavefront alone, and with a
//           value row to encode (page mode, or VB = 2 / 4) the other three
//           group-encode the values meanwhile (v_encode16, the same bits as
//           v_encode_rows), reading them from HBM while it is otherwise idle;
//   pass 2  every thread quantizes 8 channels of a token per step, writing
//           4 payload bytes.
// LDS stays under 40 KiB, so four blocks share a compute unit and their
// latency-bound phases (the Welford chains, the donor picks) overlap.
// Bit-identical to k4_encode_kernel.
constexpr int TILE_D = 128;
constexpr int TILE_T = 256;
constexpr int CH = 32;                   // tokens per staged chunk
constexpr int KPF = 1;                   // chunks in flight
constexpr int XROW = TILE_D + 8;         // u16 per staged row: 68 dwords (16-byte aligned rows, distinct banks)
// sealed blocks stream by direct global -> LDS loads into NBUF chunk buffers
// (unpadded rows), NBUF - 1 chunks in flight while one is processed
constexpr int NBUF_DMA = 4;

// s_waitcnt vmcnt(2 * ahead) lgkmcnt(0), then s_barrier: this wave's loads
// of every chunk but the `ahead` newest have landed in LDS and its LDS reads
// are done; after the barrier the same holds for every wave.  Vector memory
// operations retire in issue order, so at most 2 * ahead outstanding means
// every older load is done; stores issued after a chunk's loads only make
// the wait longer.  (A plain __syncthreads would wait for all loads in
// flight.)
__device__ __forceinline__ void wait_chunk_barrier(int ahead)
{
    switch (ahead) {
    case 0: asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    }
}

template <bool F16IN>
__device__ __forceinline__ float tile_f32(uint32_t bits16)
{
    if constexpr (F16IN) return iq_f16_to_f32((uint16_t)bits16);
    else return __uint_as_float(bits16 << 16);
}

// The eight 4-bit slots of channels 8 j .. 8 j + 7 (one packed word per
// token): per-slot constants, computed once from the role tables and pinned
// in registers (opaque to the compiler, which would otherwise rebuild them
// from the role masks at every token: four extra instructions per element).
// srcc[e] is the channel whose value slot e encodes: its own, or for a donor
// slot its source's.
struct K4Slots {
    float scl[8], rscl[8], top[8], bias[8];
    uint32_t shift[8];
    int srcc[8];

    __device__ __forceinline__ void init(int j, const uint8_t *is_src, const int16_t *src_of, const float *scale)
    {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int c = 8 * j + e;
            const bool hi = is_src[c];
            const int owner = src_of[c];
            const bool lo = !hi && owner >= 0;
            srcc[e] = lo ? owner : c;
            scl[e] = scale[srcc[e]];
            rscl[e] = __builtin_amdgcn_rcpf(scl[e]);
            const float lim = (hi || lo) ? 127.0f : 7.0f;
            // q + lim + 1 lands in the low mantissa bits of 1.5 * 2^23 + (lim + 1);
            // the clamp to [-lim, lim] is then [1.5 * 2^23 + 1, top]
            bias[e] = 12582912.0f + lim + 1.0f;
            top[e] = bias[e] + lim;
            shift[e] = hi ? 4u : 0u;
            asm volatile("" : "+v"(scl[e]), "+v"(rscl[e]), "+v"(top[e]), "+v"(bias[e]), "+v"(shift[e]));
        }
    }

    // The packed word of one token, v[e] the value of channel srcc[e].  The
    // reciprocal quotient p = v * rscl decides the rounding unless it is
    // within 2^-13 of a half-integer, where the IEEE quotient decides.  Below
    // |p| = 256, p is within 2^-14 of the IEEE quotient (v_rcp_f32 is within
    // 1 ulp, plus the quotient's own half ulp), so no rounding can differ
    // outside that band; beyond it every code clamps to +-lim either way.
    // One fma rounds p onto the integer grid of bias = 1.5 * 2^23 + lim + 1
    // (spacing 1 there): y = bias + rint(p) exactly, whose low mantissa bits
    // are the code plus lim + 1 once y is clamped to bias +- lim.  A second
    // fma gives p - rint(p) with one rounding for the band test, one max
    // over the lane's eight distances; the rare lanes inside it redo only
    // the slots that are.
    __device__ __forceinline__ uint32_t word(const float (&v)[8]) const
    {
        float y[8], q[8];
        float dmax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            y[e] = __builtin_fmaf(v[e], rscl[e], bias[e]);
            q[e] = __fsub_rn(y[e], bias[e]);                 // rint(p), exact
            dmax = fmaxf(dmax, fabsf(__builtin_fmaf(v[e], rscl[e], -q[e])));
        }
        constexpr float band = 0.5f - 0x1p-13f;
        if (__builtin_expect(dmax >= band, 0)) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (fabsf(__builtin_fmaf(v[e], rscl[e], -q[e])) >= band)
                    y[e] = __fadd_rn(rintf(v[e] / scl[e]), bias[e]);
        }
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float yc = __builtin_amdgcn_fmed3f(y[e], 12582913.0f, top[e]);
            w |= __builtin_amdgcn_ubfe(__float_as_uint(yc), shift[e], 4) << (4 * e);
        }
        return w;
    }
};

// The V2 codes and group parameters of token t of head h in a page (value
// lanes of 16 channels, vj = 0 .. 7, four lanes per 64-channel group).
__device__ __forceinline__ void store_page_values(const K4Args &a, uint8_t *page, int64_t h, int T, int t, int vj,
                                                  uint32_t code, uint16_t off_h, uint16_t sc_h)
{
    const int64_t r = h * T + t;
    __builtin_nontemporal_store(code, (uint32_t *)(page + a.off_vpay + r * 32) + vj);
    if ((vj & 3) == 0) ((uint16_t *)(page + a.off_voff))[r * 2 + (vj >> 2)] = off_h;
    if ((vj & 3) == 3) ((uint16_t *)(page + a.off_vscale))[r * 2 + (vj >> 2)] = sc_h;
}

// NCH > 0: the block length is NCH chunks (a sealed cache block), known at
// compile time, so the chunk loops unroll without branches and each load is
// waited for exactly when its chunk is stored (a branch around loads makes
// the compiler wait for all of them).  NCH = 0: any T <= 256.
// PAGES: the row goes into a physical page, values V2 with 64-channel groups.
// VB = 2 / 4 (not PAGES): the row's values are encoded too, VB bits with
// 16 * VGL-channel groups, into the outputs of iq_v_quantize.
// The body of one workgroup: row (b, h) of the encode `a`; `lin` is the
// workgroup's linear index (neighbouring blocks alternate their wave roles).
template <bool F16IN, int NCH, bool PAGES = false, int VB = 0, int VGL = 4>
__device__ __forceinline__ void k4_tile_body(const K4Args &a, int64_t b, int64_t h, int lin)
{
    constexpr int VBITS = PAGES ? 2 : VB;
    constexpr int GLV = PAGES ? 4 : VGL;
    static_assert(VBITS == 0 || VBITS == 2 || VBITS == 4, "value bits");
    static_assert(GLV == 2 || GLV == 4 || GLV == 8, "value group");
    constexpr bool DMA = NCH > 0;
    constexpr int NBUF = DMA ? NBUF_DMA : 2;
    constexpr int ROWLEN = DMA ? TILE_D : XROW;       // u16 per staged row
    static_assert(!DMA || (NBUF >= 2 && NBUF <= 4), "chunk buffers");
    __shared__ __attribute__((aligned(16))) uint16_t s_x[NBUF][CH * ROWLEN];
    __shared__ double s_rcp[TILE_T];    // RN(1 / n), n = 1 .. T
    __shared__ __attribute__((aligned(16))) float s_sal[TILE_D], s_smean[TILE_D], s_err[TILE_D], s_amax[TILE_D],
        s_scale[TILE_D];
    __shared__ int16_t s_src_of[TILE_D];
    __shared__ uint8_t s_is_src[TILE_D];
    __shared__ int16_t s_src[TILE_D / 2], s_don[TILE_D / 2];
    __shared__ __attribute__((aligned(16))) uint64_t s_key[TILE_D];
    __shared__ __attribute__((aligned(16))) int s_part[K4_THREADS];
    __shared__ __attribute__((aligned(16))) uint8_t s_flag[TILE_D];
    __shared__ int16_t s_list[TILE_D / 2];
    __shared__ int s_bad;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = b * a.H + h;
    uint8_t *page = nullptr;
    __shared__ int16_t s_role[TILE_D];
    if constexpr (PAGES) {
        if (b == 0 && h == 0 && threadIdx.x < 3) a.clear[threadIdx.x] = 0;
        const int64_t id = a.id_bytes == 8 ? ((const int64_t *)a.ids)[b] : (int64_t)((const int32_t *)a.ids)[b];
        if (id < 0 || id >= a.pool_pages) {             // uniform: before any barrier or load
            if (threadIdx.x == 0) *a.badid = 1;
            return;
        }
        page = a.pool + id * a.page_bytes;
        if (threadIdx.x < TILE_D) s_role[threadIdx.x] = -1;
    }
    const int64_t prow = PAGES && a.page_rows ? a.page_rows[b] : -1;
    const int64_t xoff = prow >= 0 ? prow * a.st : b * a.sb, voff = prow >= 0 ? prow * a.vst : b * a.vsb;
    const uint16_t *xr = (const uint16_t *)a.x + xoff + h * a.sh;
    const int T = NCH > 0 ? NCH * CH : (int)a.T;
    const int stride = (int)min(a.stride, (int64_t)TILE_T);   // a larger stride samples token 0 only
    const int ns = (T + stride - 1) / stride;
    const int nch = (T + CH - 1) / CH;

    // chunk staging: thread tid moves segments tid and tid + 256 (row i / 16,
    // 8 channels at 8 (i % 16)); rows past T are clamped copies, never read.
    // Three chunks stay in flight in registers (about 24 KiB per block), which
    // is what covers the load latency while every block streams at once.
    u32x4_t seg[KPF][2];
    auto load_chunk = [&](int ch, u32x4_t (&sg)[2]) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = tid + K4_THREADS * k;
            const int t = min(ch * CH + (i >> 4), T - 1);
            sg[k] = *(const u32x4_t *)(xr + (int64_t)t * a.st + 8 * (i & 15));
        }
    };
    auto store_chunk = [&](const u32x4_t (&sg)[2], int buf) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = tid + K4_THREADS * k;
            *(u32x4_t *)(s_x[buf] + (i >> 4) * ROWLEN + 8 * (i & 15)) = sg[k];
        }
    };
    // direct loads of chunk ch into buffer ch % NBUF: each wave fills its two
    // 1 KiB quarters (64 lanes x 16 bytes, 4 rows each); every row is a whole
    // block row, so no clamping
    // LDS byte address of the staging buffers
    const uint32_t s_x_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)&s_x[0][0];
    // lane byte offset of segment 128 wave + lane within a chunk (rows 4 on
    // for the second load); the chunk base is wave-uniform
    const uint32_t dma_off = (uint32_t)(((8 * wave + (lane >> 4)) * (int)a.st + 8 * (lane & 15)) * 2);
    auto dma_chunk = [&](int ch) {
        const char *cb = (const char *)xr + (int64_t)ch * CH * a.st * 2;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t dst = s_x_lds + (uint32_t)((ch % NBUF) * CH * ROWLEN * 2 + 16 * (128 * wave + 64 * k));
            lds_load16(cb, dma_off + (uint32_t)(k * 4 * (int)a.st * 2), dst);
        }
    };
    auto buf_of = [&](int ch) -> const uint16_t * { return s_x[DMA ? ch % NBUF : ch & 1]; };
    // registers: chunks 0..KPF-1 are loaded and chunk 0 is in LDS buffer 0;
    // direct loads: chunks 0..NBUF-2 are requested
    auto start_stream = [&]() {
        if constexpr (DMA) {
#pragma unroll
            for (int r = 0; r < NBUF - 1; ++r)
                if (r < NCH) dma_chunk(r);
        } else {
#pragma unroll
            for (int r = 0; r < KPF; ++r)
                if (r < nch) load_chunk(r, seg[r]);
        }
    };
    // visits chunks in order, chunk ch in buf_of(ch) during body(ch)
    auto stream = [&](auto &&body) {
        if constexpr (DMA) {
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) {
                // requested so far: chunks 0 .. ch + NBUF - 2
                wait_chunk_barrier(min(NBUF - 2, NCH - 1 - ch));
                // every wave is past body(ch - 1): its buffer takes chunk ch + NBUF - 1
                if (ch + NBUF - 1 < NCH) dma_chunk(ch + NBUF - 1);
                body(ch);
            }
        } else {
            for (int c0 = 0; c0 < nch; c0 += KPF) {
#pragma unroll
                for (int r = 0; r < KPF; ++r) {
                    const int ch = c0 + r;
                    if (ch < nch) {
                        if (ch + KPF < nch) load_chunk(ch + KPF, seg[r]);   // seg[r] already sits in LDS
                        body(ch);
                        if (ch + 1 < nch) store_chunk(seg[(r + 1) % KPF], (ch + 1) & 1);
                        __syncthreads();
                    }
                }
            }
        }
    };

    start_stream();
    if (NCH == 0 && tid < T) s_rcp[tid] = 1.0 / (double)(tid + 1);
    if (tid == 0) s_bad = 0;
    if constexpr (!DMA) store_chunk(seg[0], 0);
    __syncthreads();

    // ---- pass 1: statistics.  Two waves run the Welford chains (channel
    // tid & 127) and two the sums; which pair does which alternates between
    // neighbouring blocks, so that the blocks sharing a compute unit spread
    // the fp64 chains over all four SIMDs instead of stacking them on two.
    const bool welford = ((tid >> 7) ^ ((lin >> 8) & 1)) == 0;
    // The Welford chains are the critical path of pass 1 (the sums waves
    // then wait at every chunk barrier), so their waves issue first.
    if (welford && a.min_error) __builtin_amdgcn_s_setprio(2);
    double mean = 0.0, m2 = 0.0;                  // Welford waves
    IqCascade sa, sm;                             // sums waves
    sa.init(ns);
    sm.init(ns);
    uint32_t amax_bits = 0;
    int next_sample = 0;
    const int c1 = tid & (TILE_D - 1);
    stream([&](int ch) {
        const uint16_t *xs = buf_of(ch) + c1;
        const int t0 = ch * CH, nt = min(CH, T - t0);
        if (welford) {
            if (a.min_error) {
                auto step = [&](float xf, double y, int t) {
                    const double dv = (double)xf;
                    const double delta = __dsub_rn(dv, mean);
                    const double q0 = __dmul_rn(delta, y);
                    const double r = __builtin_fma(-q0, (double)(t + 1), delta);
                    mean = __dadd_rn(mean, __builtin_fma(r, y, q0));
                    const double nd = __dsub_rn(dv, mean);
                    m2 = __dadd_rn(m2, __dmul_rn(delta, nd));
                };
                // A sealed block's counts n = t + 1 are compile-time constants, and
                // so are y_hi = RN(1/n) and y_lo = RN((1 - y_hi n) / n) (the residual
                // 1 - y_hi n is exact).  delta / n is then one fma:
                // RN(delta y_hi + RN(delta y_lo)).  A quotient by an integer n <= 256
                // is never a midpoint between doubles and lies at least ulp / 512
                // from one (its odd part would need 54 bits), while
                // delta y_hi + RN(delta y_lo) is within 2^-105 |delta / n|, i.e.
                // 2^-52 ulp, of it: the fma returns the correctly rounded quotient,
                // with one dependent operation fewer than the remainder correction.
                auto step_c = [&](float xf, int t) {
                    const double n = (double)(t + 1);
                    double yh = 1.0 / n;
                    double yl = __builtin_fma(-yh, n, 1.0) / n;
                    asm("" : "+s"(yh), "+s"(yl));      // scalar operands of the mul and the fma
                    const double dv = (double)xf;
                    const double delta = __dsub_rn(dv, mean);
                    mean = __dadd_rn(mean, __builtin_fma(delta, yh, __dmul_rn(delta, yl)));
                    const double nd = __dsub_rn(dv, mean);
                    m2 = __dadd_rn(m2, __dmul_rn(delta, nd));
                };
                if constexpr (NCH > 0) {
                    // LDS reads of the next eight tokens in flight while the
                    // current eight dependent steps run
                    float cur[8], nxt[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) cur[u] = tile_f32<F16IN>(xs[u * ROWLEN]);
#pragma unroll
                    for (int g = 0; g < CH; g += 8) {
                        const int gn = g + 8 < CH ? g + 8 : g;
#pragma unroll
                        for (int u = 0; u < 8; ++u) nxt[u] = tile_f32<F16IN>(xs[(gn + u) * ROWLEN]);
#pragma unroll
                        for (int u = 0; u < 8; ++u) step_c(cur[u], t0 + g + u);
#pragma unroll
                        for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
                    }
                } else if (nt == CH) {
                    // LDS reads of the next eight tokens in flight while the
                    // current eight dependent steps run
                    float cur[8], nxt[8];
                    double ycur[8], ynxt[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        cur[u] = tile_f32<F16IN>(xs[u * ROWLEN]);
                        ycur[u] = s_rcp[t0 + u];
                    }
#pragma unroll
                    for (int g = 0; g < CH; g += 8) {
                        const int gn = g + 8 < CH ? g + 8 : g;
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            nxt[u] = tile_f32<F16IN>(xs[(gn + u) * ROWLEN]);
                            ynxt[u] = s_rcp[t0 + gn + u];
                        }
#pragma unroll
                        for (int u = 0; u < 8; ++u) step(cur[u], ycur[u], t0 + g + u);
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            cur[u] = nxt[u];
                            ycur[u] = ynxt[u];
                        }
                    }
                } else {
                    for (int u = 0; u < nt; ++u) step(tile_f32<F16IN>(xs[u * ROWLEN]), s_rcp[t0 + u], t0 + u);
                }
            }
        } else {
            // |x| as 16-bit integers: for finite values their order is the
            // order of the magnitudes, and inf / NaN sort above every finite one
            if (nt == CH) {
#pragma unroll
                for (int u = 0; u < CH; ++u) amax_bits = max(amax_bits, (uint32_t)xs[u * ROWLEN] & 0x7fffu);
            } else {
                for (int u = 0; u < nt; ++u) amax_bits = max(amax_bits, (uint32_t)xs[u * ROWLEN] & 0x7fffu);
            }
            // the samples r * stride that fall in this chunk, in order
            for (; next_sample < t0 + nt; next_sample += stride) {
                const float v = tile_f32<F16IN>(xs[(next_sample - t0) * ROWLEN]);
                sa.add(fabsf(v));
                sm.add(v);
            }
        }
    });
    if (welford) {
        if (a.min_error) {
            s_err[c1] = (float)(m2 / (double)T);      // var; the mean term is added below
            s_smean[c1] = (float)mean;                // full mean, replaced below
        }
    } else {
        s_amax[c1] = tile_f32<F16IN>(amax_bits);
        s_sal[c1] = sa.finish() / (float)ns;
        if (amax_bits >= (F16IN ? 0x7c00u : 0x7f80u)) s_bad = 1;     // an inf or NaN in the channel
        // stash the sampled mean until the Welford waves are done with s_smean
        s_scale[c1] = sm.finish() / (float)ns;
    }
    // A sealed block's last NBUF chunks are still in the buffers after pass 1
    // and pass 2 quantizes them first (RESIDENT), reloading the others into
    // the buffers they free; otherwise the first chunks of pass 2 load during
    // the selection (once every wave is done with pass 1's buffers).
    constexpr bool RESIDENT = DMA && NCH == 2 * NBUF;
    __syncthreads();
    if constexpr (!RESIDENT) start_stream();

    // ---- values (VBITS > 0), encoded by three wavefronts while the fourth
    // makes the sequential donor picks, with the row's HBM reads in that otherwise
    // idle stretch.  Thread vt of the three value wavefronts takes channels 16 vj .. 16 vj + 15
    // of token vtok0 + 24 it in iteration it (192 threads = 24 tokens), so a
    // group's GLV lanes are adjacent lanes of one wavefront.  A sealed block
    // (11 iterations) issues its first VPF iterations' loads here, before
    // the ranks; the rest run VPF iterations ahead.
    constexpr int VT = K4_THREADS - 64;
    constexpr int VIT = NCH > 0 ? (NCH * CH * 8 + VT - 1) / VT : 1;
    constexpr int VPF = 4;
    // The picking wavefront rotates between the workgroups that share a
    // compute unit (linear indices 256 apart): each SIMD then holds one
    // picking wavefront and three encoding values, instead of one SIMD
    // holding every picker while its VALU idles.  vtid is the thread's index
    // in that rotated order (virtual wave 0 picks).
    const int vtid = (tid + 64 * ((lin >> 8) & 3)) & (K4_THREADS - 1), vwave = vtid >> 6;
    const int vt = vtid - 64, vj = vt & 7, vtok0 = vt >> 3;
    u32x4_t vraw[NCH > 0 ? VIT : 1][2];
    auto vload = [&](int it, u32x4_t(&r)[2]) {
        const int t = min(vtok0 + 24 * it, T - 1);
        const u32x4_t *p = (const u32x4_t *)(a.v + voff + h * a.vsh + (int64_t)t * a.vst + 16 * vj);
        r[0] = __builtin_nontemporal_load(p);
        r[1] = __builtin_nontemporal_load(p + 1);
    };
    auto vencode = [&](int it, const u32x4_t(&r)[2], bool &vbad) {
        const int t = vtok0 + 24 * it;
        const bool live = t < T;
        uint32_t code[VBITS > 0 ? VBITS / 2 : 1];
        uint16_t off_h, sc_h;
        if constexpr (VBITS > 0) v_encode16<F16IN, VBITS, GLV>(r, live, code, off_h, sc_h, vbad);
        if (VBITS > 0 && live) {
            if constexpr (PAGES) {
                store_page_values(a, page, h, T, t, vj, code[0], off_h, sc_h);
            } else {
                constexpr int PB = TILE_D * (VBITS > 0 ? VBITS : 2) / 8;   // payload bytes per token
                constexpr int GROUPS = 8 / GLV;
                const int64_t vr = row * T + t;
                if constexpr (VBITS == 2) {
                    __builtin_nontemporal_store(code[0], (uint32_t *)(a.vpayload + vr * PB) + vj);
                } else {
                    typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;
                    ((u32x2_t *)(a.vpayload + vr * PB))[vj] = u32x2_t{code[0], code[VBITS / 2 - 1]};
                }
                if (vj % GLV == 0) a.voffsets[vr * GROUPS + vj / GLV] = off_h;
                if (vj % GLV == GLV - 1) a.vscales[vr * GROUPS + vj / GLV] = sc_h;
            }
        }
    };
    if constexpr (VBITS > 0 && NCH > 0) {
        if (vwave > 0) {
#pragma unroll
            for (int it = 0; it < VPF; ++it) vload(it, vraw[it]);
        }
    }

    if (tid < TILE_D) {
        const float smean = s_scale[tid];
        if (a.min_error) {
            const float diff = __fsub_rn(s_smean[tid], smean);
            s_err[tid] = __fadd_rn(s_err[tid], __fmul_rn(diff, diff));
        }
        s_smean[tid] = smean;
    }
    __syncthreads();

    // the sequential donor picks on the picking wavefront hold up the whole block: top priority
    if (vwave == 0) __builtin_amdgcn_s_setprio(3);
    else __builtin_amdgcn_s_setprio(0);
    iq_select_tile128(s_sal, a.min_error ? s_err : nullptr, (int)a.count, s_src, s_don, s_is_src, s_src_of,
                      s_key, s_part, s_flag, s_list, vtid);
    if constexpr (VBITS > 0) {
        if (vwave > 0) {
            bool vbad = false;
            if constexpr (NCH > 0) {
#pragma unroll
                for (int it = 0; it < VIT; ++it) {
                    if (it + VPF < VIT) vload(it + VPF, vraw[it + VPF]);
                    vencode(it, vraw[it], vbad);
                }
            } else {
                const int nit = (T * 8 + VT - 1) / VT;
                for (int it = 0; it < nit; ++it) {
                    vload(it, vraw[0]);
                    vencode(it, vraw[0], vbad);
                }
            }
            if (__ballot(vbad) != 0 && lane == 0) atomicOr(a.vbad, 1);
        }
    }
    __builtin_amdgcn_s_setprio(1);
    __syncthreads();

    const float flt_min = 1.17549435e-38f;
    if (tid < TILE_D) {
        const float s = s_amax[tid] / (s_is_src[tid] ? 127.0f : 7.0f);
        const float sc = s < flt_min ? flt_min : s;
        s_scale[tid] = sc;
        if constexpr (PAGES) ((float *)(page + a.off_kscale))[h * TILE_D + tid] = sc;
        else a.scales[row * TILE_D + tid] = sc;
    }
    if (tid < a.count) {
        if constexpr (PAGES) {
            // page role map: the donor channel for a source, -2 - k for donor k
            s_role[s_src[tid]] = (int16_t)s_don[tid];
            s_role[s_don[tid]] = (int16_t)(-2 - tid);
            ((float *)(page + a.off_kpad))[h * a.count + tid] = s_smean[s_don[tid]];
        } else {
            store_desc(a.src, row * a.count + tid, s_src[tid], a.desc_bytes);
            store_desc(a.don, row * a.count + tid, s_don[tid], a.desc_bytes);
            a.padding[row * a.count + tid] = s_smean[s_don[tid]];
        }
    }
    if (tid == 0 && s_bad) atomicOr(a.bad, 1);
    if constexpr (!DMA) store_chunk(seg[0], 0);
    __syncthreads();

    // ---- pass 2: quantize; thread owns channels 8 j .. 8 j + 7 of tokens
    // t0 + 8 wave + tq and t0 + 8 wave + tq + 4 of every chunk
    const int j = lane & 15, tq = lane >> 4;
    K4Slots slots;
    slots.init(j, s_is_src, s_src_of, s_scale);
    // xe[e]: LDS address of slot e's value in row 8 wave + tq of buffer 0;
    // every other row and buffer is a constant offset from it
    const uint16_t *xe[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) xe[e] = &s_x[0][0] + (8 * wave + tq) * ROWLEN + slots.srcc[e];
    if constexpr (PAGES) {
        if (tid < TILE_D) ((int16_t *)(page + a.off_kmap))[h * TILE_D + tid] = s_role[tid];
    }
    uint32_t *out = PAGES ? (uint32_t *)(page + a.off_kpay + h * (int64_t)T * (TILE_D / 2))
                          : (uint32_t *)(a.payload + row * (int64_t)T * (TILE_D / 2));
    // chunks NCH - NBUF .. NCH - 1 from the buffers pass 1 left them in, then
    // chunk c < NCH - NBUF, loaded into buffer c % NBUF once every wave is
    // done with the resident chunk c + NBUF there (issued NBUF - 1 chunks
    // ahead of its use; waits as in stream(): vector memory operations retire
    // in order, and the stores issued in between only lengthen them)
    auto stream2 = [&](auto &&body) {
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int ch = k < NBUF ? NCH - NBUF + k : k - NBUF;
            if (k >= NBUF) wait_chunk_barrier(min(NBUF - 2, NCH - 1 - k));
            else if (k > 0) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (k > 0 && k <= NBUF) dma_chunk(k - 1);
            body(ch);
        }
    };
    auto pass2 = [&](int ch) {
        const int t0 = ch * CH;
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int tl = 8 * wave + 4 * it + tq, t = t0 + tl;
            if (t < T) {
                const int off = (DMA ? ch % NBUF : ch & 1) * CH * ROWLEN + 4 * it * ROWLEN;
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = tile_f32<F16IN>(xe[e][off]);
                __builtin_nontemporal_store(slots.word(v), &out[t * (TILE_D / 8) + j]);
            }
        }
    };
    if constexpr (RESIDENT) stream2(pass2);
    else stream(pass2);
}

// grid (blocks, heads): no 64-bit division for the row's coordinates
template <bool F16IN, int NCH, bool PAGES = false, int VB = 0, int VGL = 4>
__global__ __launch_bounds__(K4_THREADS, 4) void k4_encode_tile(K4Args a)
{
    k4_tile_body<F16IN, NCH, PAGES, VB, VGL>(a, blockIdx.x, blockIdx.y, (int)(blockIdx.x + gridDim.x * blockIdx.y));
}

// Keys and values of the same blocks, both K4, in one launch: grid (blocks,
// 2 H), rows h < H of the keys `ak`, the others of the values `av`.
template <bool F16IN, int NCH>
__global__ __launch_bounds__(K4_THREADS, 4) void k4_encode_pair(K4Args ak, K4Args av)
{
    const bool val = (int64_t)blockIdx.y >= ak.H;
    const K4Args a = val ? av : ak;
    k4_tile_body<F16IN, NCH>(a, blockIdx.x, val ? blockIdx.y - ak.H : blockIdx.y,
                             (int)(blockIdx.x + gridDim.x * blockIdx.y));
}

// Pages of T = 16 or 32 tokens: one wavefront encodes one (page, head) row,
// keys and values, and a workgroup holds four rows (pages 4 blockIdx.x + wave
// of head blockIdx.y) that share nothing, so there is no workgroup barrier.
// A short row keeps the serial phases of the 256-thread tile encoder (the
// donor selection is the same 16 picks for 16 tokens as for 256) while its
// other waves idle; here each wavefront runs its own row from start to end
// and a compute unit interleaves twenty rows.  The arithmetic and its order
// are the tile encoder's, so the page bytes are the same:
//   lane l owns channels 2 l and 2 l + 1 for the statistics (fp64 Welford
//   with the exact reciprocals 1 / n, amax as 16-bit magnitudes, sampled sums
//   in torch's cascade order), iq_select_wave128 makes the selection, lane
//   (j, tq) = (l % 16, l / 16) packs channels 8 j .. 8 j + 7 of tokens
//   tq + 4 i, and lane (vj, vt) = (l % 8, l / 8) encodes channels
//   16 vj .. 16 vj + 15 of value tokens vt + 8 i.
// Lanes read LDS words other lanes of the same wavefront wrote: a
// wavefront's LDS operations complete in order, so the wavefront-scope
// fences emit nothing and only keep the compiler from reordering.
template <bool F16IN, int T>
__global__ __launch_bounds__(K4_THREADS) void k4_encode_page_rows(K4Args a, int64_t n_pages)
{
    static_assert(T == 16 || T == 32, "short pages");
    constexpr int ROW = TILE_D + 8;            // u16 per staged token row
    constexpr int KSEG = T * (TILE_D / 8) / 64; // 16-byte key segments per lane
    constexpr int VIT = T / 8;                 // value tokens per lane
    __shared__ __attribute__((aligned(16))) uint16_t s_x[4][T * ROW];
    __shared__ __attribute__((aligned(8))) float s_sal[4][TILE_D], s_err[4][TILE_D], s_mean[4][TILE_D];
    __shared__ int16_t s_src[4][TILE_D / 2], s_don[4][TILE_D / 2], s_src_of[4][TILE_D], s_role[4][TILE_D];
    __shared__ int16_t s_list[4][TILE_D / 2];
    __shared__ uint8_t s_is_src[4][TILE_D];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t b = (int64_t)blockIdx.x * 4 + wave, h = blockIdx.y;
    if (blockIdx.x == 0 && h == 0 && threadIdx.x < 3) a.clear[threadIdx.x] = 0;
    if (b >= n_pages) return;                  // wave-uniform, as the page check below
    const int64_t id = a.id_bytes == 8 ? ((const int64_t *)a.ids)[b] : (int64_t)((const int32_t *)a.ids)[b];
    if (id < 0 || id >= a.pool_pages) {
        if (lane == 0) *a.badid = 1;
        return;
    }
    uint8_t *const page = a.pool + id * a.page_bytes;
    const int64_t prow = a.page_rows ? a.page_rows[b] : -1;
    const uint16_t *const xr = (const uint16_t *)a.x + (prow >= 0 ? prow * a.st : b * a.sb) + h * a.sh;
    const uint16_t *const vr = a.v + (prow >= 0 ? prow * a.vst : b * a.vsb) + h * a.vsh;

    // every load of the row first: key segment i = lane + 64 k is token i / 16,
    // channels 8 (i % 16) ..; value lane (vj, vt) reads 16 channels of token vt + 8 it
    const int vj = lane & 7, vt = lane >> 3;
    u32x4_t kseg[KSEG], vraw[VIT][2];
#pragma unroll
    for (int k = 0; k < KSEG; ++k) {
        const int i = lane + 64 * k;
        kseg[k] = *(const u32x4_t *)(xr + (int64_t)(i >> 4) * a.st + 8 * (i & 15));
    }
#pragma unroll
    for (int it = 0; it < VIT; ++it) {
        const u32x4_t *p = (const u32x4_t *)(vr + (int64_t)(vt + 8 * it) * a.vst + 16 * vj);
        vraw[it][0] = __builtin_nontemporal_load(p);
        vraw[it][1] = __builtin_nontemporal_load(p + 1);
    }
    uint16_t *const xs = s_x[wave];
#pragma unroll
    for (int k = 0; k < KSEG; ++k) {
        const int i = lane + 64 * k;
        *(u32x4_t *)(xs + (i >> 4) * ROW + 8 * (i & 15)) = kseg[k];
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");

    // ---- statistics of channels 2 lane and 2 lane + 1
    double mean[2] = {0.0, 0.0}, m2[2] = {0.0, 0.0};
    uint32_t amax_bits[2] = {0u, 0u};
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const uint32_t w = *(const uint32_t *)(xs + t * ROW + 2 * lane);
        // delta / n as in the tile encoder's step_c: one fma with the
        // compile-time pair RN(1/n), RN((1 - RN(1/n) n) / n)
        const double n = (double)(t + 1);
        const double yh = 1.0 / n;
        const double yl = __builtin_fma(-yh, n, 1.0) / n;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t u = e ? w >> 16 : w & 0xffffu;
            amax_bits[e] = max(amax_bits[e], u & 0x7fffu);
            const double dv = (double)tile_f32<F16IN>(u);
            const double delta = __dsub_rn(dv, mean[e]);
            mean[e] = __dadd_rn(mean[e], __builtin_fma(delta, yh, __dmul_rn(delta, yl)));
            m2[e] = __dadd_rn(m2[e], __dmul_rn(delta, __dsub_rn(dv, mean[e])));
        }
    }
    const int stride = (int)min(a.stride, (int64_t)TILE_T);   // a larger stride samples token 0 only
    const int ns = (T + stride - 1) / stride;
    IqCascade sa[2], sm[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        sa[e].init(ns);
        sm[e].init(ns);
    }
    for (int t = 0; t < T; t += stride) {
        const uint32_t w = *(const uint32_t *)(xs + t * ROW + 2 * lane);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float v = tile_f32<F16IN>(e ? w >> 16 : w & 0xffffu);
            sa[e].add(fabsf(v));
            sm[e].add(v);
        }
    }
    float amax[2];
    bool kbad = false;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int c = 2 * lane + e;
        const float smean = sm[e].finish() / (float)ns;
        const float diff = __fsub_rn((float)mean[e], smean);
        s_err[wave][c] = __fadd_rn((float)(m2[e] / (double)T), __fmul_rn(diff, diff));
        s_sal[wave][c] = sa[e].finish() / (float)ns;
        s_mean[wave][c] = smean;
        amax[e] = tile_f32<F16IN>(amax_bits[e]);
        kbad |= amax_bits[e] >= (F16IN ? 0x7c00u : 0x7f80u);   // an inf or NaN in the channel
    }
    if (__ballot(kbad) != 0 && lane == 0) atomicOr(a.bad, 1);

    // ---- values, while the selection's inputs settle
    bool vbad = false;
#pragma unroll
    for (int it = 0; it < VIT; ++it) {
        uint32_t code[1];
        uint16_t off_h, sc_h;
        v_encode16<F16IN, 2, 4>(vraw[it], true, code, off_h, sc_h, vbad);
        store_page_values(a, page, h, T, vt + 8 * it, vj, code[0], off_h, sc_h);
    }
    if (__ballot(vbad) != 0 && lane == 0) atomicOr(a.vbad, 1);

    // ---- selection, scales, role map and padding
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const int count = (int)a.count;
    iq_select_wave128(s_sal[wave], s_err[wave], count, s_src[wave], s_don[wave], s_is_src[wave], s_src_of[wave],
                      s_list[wave]);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const float flt_min = 1.17549435e-38f;
    float *const kscale = (float *)(page + a.off_kscale) + h * TILE_D;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int c = 2 * lane + e;
        const float s = amax[e] / (s_is_src[wave][c] ? 127.0f : 7.0f);
        const float sc = s < flt_min ? flt_min : s;
        s_sal[wave][c] = sc;                   // the saliencies are spent: scales from here on
        kscale[c] = sc;
        s_role[wave][c] = -1;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    if (lane < count) {
        // page role map: the donor channel for a source, -2 - k for donor k
        const int s = s_src[wave][lane], d = s_don[wave][lane];
        s_role[wave][s] = (int16_t)d;
        s_role[wave][d] = (int16_t)(-2 - lane);
        ((float *)(page + a.off_kpad))[h * count + lane] = s_mean[wave][d];
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    int16_t *const kmap = (int16_t *)(page + a.off_kmap) + h * TILE_D;
    kmap[2 * lane] = s_role[wave][2 * lane];
    kmap[2 * lane + 1] = s_role[wave][2 * lane + 1];

    // ---- 4-bit slots
    const int j = lane & 15, tq = lane >> 4;
    K4Slots slots;
    slots.init(j, s_is_src[wave], s_src_of[wave], s_sal[wave]);
    uint32_t *const out = (uint32_t *)(page + a.off_kpay + h * (int64_t)T * (TILE_D / 2));
#pragma unroll
    for (int it = 0; it < T / 4; ++it) {
        const int t = tq + 4 * it;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = tile_f32<F16IN>(xs[t * ROW + slots.srcc[e]]);
        __builtin_nontemporal_store(slots.word(v), &out[t * (TILE_D / 8) + j]);
    }
}

struct SelectArgs {
    const float *sal, *err;
    int64_t D, count;
    int64_t *src, *don;
};

__global__ __launch_bounds__(64) void reuse_map_kernel(SelectArgs a)
{
    __shared__ float s_sal[IQ_MAXD];
    __shared__ float s_err[IQ_MAXD];
    __shared__ int16_t s_src_of[IQ_MAXD];
    __shared__ uint8_t s_is_src[IQ_MAXD];
    __shared__ int16_t s_src[IQ_MAXD / 2];
    __shared__ int16_t s_don[IQ_MAXD / 2];
    const int64_t row = blockIdx.x;
    for (int64_t c = threadIdx.x; c < a.D; c += 64) {
        s_sal[c] = a.sal[row * a.D + c];
        if (a.err) s_err[c] = a.err[row * a.D + c];
    }
    __syncthreads();
    iq_select_wave(s_sal, a.err ? s_err : nullptr, (int)a.D, (int)a.count, s_src, s_don, s_is_src, s_src_of);
    __syncthreads();
    for (int64_t i = threadIdx.x; i < a.count; i += 64) {
        a.src[row * a.count + i] = s_src[i];
        a.don[row * a.count + i] = s_don[i];
    }
}

// D = 128: one wavefront per row with the radix top-k selection of the page
// row encoder (iq_select_wave128), the same picks as iq_select_wave.
__global__ __launch_bounds__(64) void reuse_map128_kernel(SelectArgs a)
{
    __shared__ float s_sal[128], s_err[128];
    __shared__ int16_t s_src_of[128], s_src[64], s_don[64], s_list[64];
    __shared__ uint8_t s_is_src[128];
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x;
    s_sal[lane] = a.sal[row * 128 + lane];
    s_sal[64 + lane] = a.sal[row * 128 + 64 + lane];
    if (a.err) {
        s_err[lane] = a.err[row * 128 + lane];
        s_err[64 + lane] = a.err[row * 128 + 64 + lane];
    }
    __syncthreads();
    iq_select_wave128(s_sal, a.err ? s_err : nullptr, (int)a.count, s_src, s_don, s_is_src, s_src_of, s_list);
    __syncthreads();
    if (lane < a.count) {
        a.src[row * a.count + lane] = s_src[lane];
        a.don[row * a.count + lane] = s_don[lane];
    }
}

}  // namespace

namespace {

// the tile encoder's layout: 16-bit channel-contiguous rows of 128 channels,
// 16-byte aligned, at most 256 tokens, 32-bit lane offsets within a chunk
bool tile_ok(const void *x, int dtype, const int64_t *s, int64_t T, int64_t D)
{
    return (dtype == IQ_BF16 || dtype == IQ_F16) && D == TILE_D && T <= TILE_T && s[3] == 1 && s[2] % 8 == 0 &&
           s[1] % 8 == 0 && s[0] % 8 == 0 && ((uintptr_t)x & 15) == 0 && s[2] >= 0 && s[2] <= (1 << 24);
}

}  // namespace

extern "C" int iq_k4_quantize(const void *x, int x_dtype, const int64_t *x_strides, int64_t B, int64_t H,
                              int64_t T, int64_t D, int64_t count, int64_t sample_stride, int min_error,
                              uint8_t *payload, float *scales, void *src, void *don, int desc_bytes,
                              float *padding, int *bad_flag, void *stream)
{
    IQ_CHECK_ARG(x && x_strides && payload && scales && bad_flag, "iq_k4_quantize: null pointer");
    IQ_CHECK_ARG(x_dtype >= IQ_F32 && x_dtype <= IQ_F64, "iq_k4_quantize: bad dtype %d", x_dtype);
    IQ_CHECK_ARG(B >= 1 && H >= 1 && T >= 1, "iq_k4_quantize: empty shape");
    IQ_CHECK_ARG(D >= 2 && D % 2 == 0 && D <= IQ_MAXD, "iq_k4_quantize: D=%lld must be even and <= %d",
                 (long long)D, IQ_MAXD);
    IQ_CHECK_ARG(count >= 0 && 2 * count <= D, "iq_k4_quantize: count=%lld out of range", (long long)count);
    IQ_CHECK_ARG(count == 0 || (src && don && padding), "iq_k4_quantize: null descriptor output");
    IQ_CHECK_ARG(sample_stride >= 1, "iq_k4_quantize: sample_stride must be positive");
    IQ_CHECK_ARG(desc_bytes == 1 || desc_bytes == 4 || desc_bytes == 8, "iq_k4_quantize: desc_bytes");
    IQ_CHECK_ARG(B * H <= 0x7fffffffLL, "iq_k4_quantize: too many rows");
    K4Args a{x, x_dtype, x_strides[0], x_strides[1], x_strides[2], x_strides[3], H, T, D, count, sample_stride,
             min_error ? 1 : 0, payload, scales, src, don, desc_bytes, padding, bad_flag};
    if (tile_ok(x, x_dtype, x_strides, T, D) && H <= 65535) {
        const dim3 grid((unsigned)B, (unsigned)H), block(K4_THREADS);
        const hipStream_t st = (hipStream_t)stream;
        if (x_dtype == IQ_F16) {
            if (T == TILE_T) hipLaunchKernelGGL((k4_encode_tile<true, TILE_T / CH>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((k4_encode_tile<true, 0>), grid, block, 0, st, a);
        } else {
            if (T == TILE_T) hipLaunchKernelGGL((k4_encode_tile<false, TILE_T / CH>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((k4_encode_tile<false, 0>), grid, block, 0, st, a);
        }
        IQ_CHECK_LAUNCH("k4_encode_tile");
        return IQ_OK;
    }
    // long rows: the per-row statistics on one workgroup each, the payload
    // spread over token tiles
    a.split = T > 4 * Q_TOKENS && B * H <= 65535 ? 1 : 0;
    hipLaunchKernelGGL(k4_encode_kernel, dim3((unsigned)(B * H)), dim3(K4_THREADS), 0, (hipStream_t)stream, a);
    IQ_CHECK_LAUNCH("k4_encode_kernel");
    if (a.split) {
        hipLaunchKernelGGL(k4_quantize_generic, dim3((unsigned)((T + Q_TOKENS - 1) / Q_TOKENS), (unsigned)(B * H)),
                           dim3(K4_THREADS), 0, (hipStream_t)stream, a);
        IQ_CHECK_LAUNCH("k4_quantize_generic");
    }
    return IQ_OK;
}

namespace {

template <bool F16IN, int VB>
void launch_kv_tile(int VGL, dim3 grid, hipStream_t st, const K4Args &a)
{
    constexpr int N = TILE_T / CH;
    switch (VGL) {
    case 2: hipLaunchKernelGGL((k4_encode_tile<F16IN, N, false, VB, 2>), grid, dim3(K4_THREADS), 0, st, a); break;
    case 4: hipLaunchKernelGGL((k4_encode_tile<F16IN, N, false, VB, 4>), grid, dim3(K4_THREADS), 0, st, a); break;
    default: hipLaunchKernelGGL((k4_encode_tile<F16IN, N, false, VB, 8>), grid, dim3(K4_THREADS), 0, st, a); break;
    }
}

}  // namespace

extern "C" int iq_kv_quantize(const void *keys, const void *values, int dtype, const int64_t *k_strides,
                              const int64_t *v_strides, int64_t B, int64_t H, int64_t T, int64_t D,
                              int64_t count, int64_t sample_stride, int min_error, uint8_t *k_payload,
                              float *k_scales, void *src, void *don, int desc_bytes, float *padding,
                              int value_bits, int value_group, uint8_t *v_payload, uint16_t *v_scales,
                              uint16_t *v_offsets, int *key_bad, int *value_bad, void *stream)
{
    IQ_CHECK_ARG(keys && values && k_strides && v_strides && k_payload && k_scales && v_payload && v_scales &&
                     v_offsets && key_bad && value_bad,
                 "iq_kv_quantize: null pointer");
    IQ_CHECK_ARG(value_bits == 2 || value_bits == 4, "iq_kv_quantize: value_bits must be 2 or 4");
    IQ_CHECK_ARG(value_group == 32 || value_group == 64 || value_group == 128,
                 "iq_kv_quantize: value_group must be 32, 64 or 128");
    auto rows16 = [](const void *p, const int64_t *s) {
        return ((uintptr_t)p & 15) == 0 && s[3] == 1 && s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0 &&
               s[2] >= 0 && s[2] <= (1 << 23);
    };
    const bool fused = (dtype == IQ_BF16 || dtype == IQ_F16) && D == TILE_D && T == TILE_T && B >= 1 &&
                       B <= 0x7fffffffLL && H >= 1 && H <= 65535 && B * H <= 0x7fffffffLL && count >= 0 &&
                       2 * count <= D && (count == 0 || (src && don && padding)) && sample_stride >= 1 &&
                       (desc_bytes == 1 || desc_bytes == 4 || desc_bytes == 8) && rows16(keys, k_strides) &&
                       rows16(values, v_strides);
    if (!fused) {
        // any other shape: the two encoders back to back on the stream
        const int rk = iq_k4_quantize(keys, dtype, k_strides, B, H, T, D, count, sample_stride, min_error,
                                      k_payload, k_scales, src, don, desc_bytes, padding, key_bad, stream);
        if (rk != IQ_OK) return rk;
        return iq_v_quantize(values, dtype, v_strides, B, H, T, D, value_bits, value_group, v_payload, v_scales,
                             v_offsets, value_bad, stream);
    }
    K4Args a{};
    a.x = keys;
    a.dt = dtype;
    a.sb = k_strides[0];
    a.sh = k_strides[1];
    a.st = k_strides[2];
    a.sc = 1;
    a.H = H;
    a.T = T;
    a.D = D;
    a.count = count;
    a.stride = sample_stride;
    a.min_error = min_error ? 1 : 0;
    a.payload = k_payload;
    a.scales = k_scales;
    a.src = src;
    a.don = don;
    a.desc_bytes = desc_bytes;
    a.padding = padding;
    a.bad = key_bad;
    a.v = (const uint16_t *)values;
    a.vsb = v_strides[0];
    a.vsh = v_strides[1];
    a.vst = v_strides[2];
    a.vbad = value_bad;
    a.vpayload = v_payload;
    a.vscales = v_scales;
    a.voffsets = v_offsets;
    const dim3 grid((unsigned)B, (unsigned)H);
    const hipStream_t st = (hipStream_t)stream;
    const int VGL = value_group / 16;
    if (dtype == IQ_F16) {
        if (value_bits == 2) launch_kv_tile<true, 2>(VGL, grid, st, a);
        else launch_kv_tile<true, 4>(VGL, grid, st, a);
    } else {
        if (value_bits == 2) launch_kv_tile<false, 2>(VGL, grid, st, a);
        else launch_kv_tile<false, 4>(VGL, grid, st, a);
    }
    IQ_CHECK_LAUNCH("k4_encode_tile (keys and values)");
    return IQ_OK;
}

extern "C" int iq_k4_quantize_kv(const void *keys, const void *values, int dtype, const int64_t *k_strides,
                                 const int64_t *v_strides, int64_t B, int64_t H, int64_t T, int64_t D, int64_t count,
                                 int64_t sample_stride, int min_error, uint8_t *k_payload, float *k_scales,
                                 void *k_src, void *k_don, float *k_padding, uint8_t *v_payload, float *v_scales,
                                 void *v_src, void *v_don, float *v_padding, int desc_bytes, int *key_bad,
                                 int *value_bad, void *stream)
{
    IQ_CHECK_ARG(keys && values && k_strides && v_strides && key_bad && value_bad, "iq_k4_quantize_kv: null pointer");
    const bool fused = tile_ok(keys, dtype, k_strides, T, D) && tile_ok(values, dtype, v_strides, T, D) && B >= 1 &&
                       B <= 0x7fffffffLL && H >= 1 && 2 * H <= 65535 && T >= 1 && count >= 0 && 2 * count <= D &&
                       sample_stride >= 1 && (desc_bytes == 1 || desc_bytes == 4 || desc_bytes == 8) &&
                       k_payload && k_scales && v_payload && v_scales &&
                       (count == 0 || (k_src && k_don && k_padding && v_src && v_don && v_padding));
    if (!fused) {
        // any other shape: the two encodes back to back on the stream
        const int rk = iq_k4_quantize(keys, dtype, k_strides, B, H, T, D, count, sample_stride, min_error, k_payload,
                                      k_scales, k_src, k_don, desc_bytes, k_padding, key_bad, stream);
        if (rk != IQ_OK) return rk;
        return iq_k4_quantize(values, dtype, v_strides, B, H, T, D, count, sample_stride, min_error, v_payload,
                              v_scales, v_src, v_don, desc_bytes, v_padding, value_bad, stream);
    }
    const K4Args ak{keys, dtype, k_strides[0], k_strides[1], k_strides[2], k_strides[3], H, T, D, count,
                    sample_stride, min_error ? 1 : 0, k_payload, k_scales, k_src, k_don, desc_bytes, k_padding,
                    key_bad};
    const K4Args av{values, dtype, v_strides[0], v_strides[1], v_strides[2], v_strides[3], H, T, D, count,
                    sample_stride, min_error ? 1 : 0, v_payload, v_scales, v_src, v_don, desc_bytes, v_padding,
                    value_bad};
    const dim3 grid((unsigned)B, (unsigned)(2 * H)), block(K4_THREADS);
    const hipStream_t st = (hipStream_t)stream;
    if (dtype == IQ_F16) {
        if (T == TILE_T) hipLaunchKernelGGL((k4_encode_pair<true, TILE_T / CH>), grid, block, 0, st, ak, av);
        else hipLaunchKernelGGL((k4_encode_pair<true, 0>), grid, block, 0, st, ak, av);
    } else {
        if (T == TILE_T) hipLaunchKernelGGL((k4_encode_pair<false, TILE_T / CH>), grid, block, 0, st, ak, av);
        else hipLaunchKernelGGL((k4_encode_pair<false, 0>), grid, block, 0, st, ak, av);
    }
    IQ_CHECK_LAUNCH("k4_encode_pair");
    return IQ_OK;
}

extern "C" int iq_reuse_map(const float *saliency, const float *donor_error, int64_t rows, int64_t D,
                            int64_t count, int64_t *src, int64_t *don, void *stream)
{
    IQ_CHECK_ARG(rows >= 0 && D >= 1 && D <= IQ_MAXD, "iq_reuse_map: D=%lld unsupported", (long long)D);
    IQ_CHECK_ARG(count >= 0 && 2 * count <= D, "iq_reuse_map: count=%lld out of range", (long long)count);
    IQ_CHECK_ARG(rows <= 0x7fffffffLL, "iq_reuse_map: too many rows");
    if (rows == 0 || count == 0) return IQ_OK;
    IQ_CHECK_ARG(saliency && src && don, "iq_reuse_map: null pointer");
    SelectArgs a{saliency, donor_error, D, count, src, don};
    if (D == 128) hipLaunchKernelGGL(reuse_map128_kernel, dim3((unsigned)rows), dim3(64), 0, (hipStream_t)stream, a);
    else hipLaunchKernelGGL(reuse_map_kernel, dim3((unsigned)rows), dim3(64), 0, (hipStream_t)stream, a);
    IQ_CHECK_LAUNCH("reuse_map_kernel");
    return IQ_OK;
}

extern "C" int iq_encode_pages(const void *keys, const void *values, int dtype, const int64_t *k_strides,
                               const int64_t *v_strides, int64_t n_pages, int64_t H, int64_t block_tokens,
                               uint8_t *pool, int64_t pool_pages, const void *page_ids, int id_bytes, int *flags,
                               int *next_flags, void *stream)
{
    return iq_encode_pages_at(keys, values, dtype, k_strides, v_strides, nullptr, n_pages, H, block_tokens, pool,
                              pool_pages, page_ids, id_bytes, flags, next_flags, stream);
}

extern "C" int iq_encode_pages_at(const void *keys, const void *values, int dtype, const int64_t *k_strides,
                                  const int64_t *v_strides, const int64_t *page_rows, int64_t n_pages, int64_t H,
                                  int64_t block_tokens, uint8_t *pool, int64_t pool_pages, const void *page_ids,
                                  int id_bytes, int *flags, int *next_flags, void *stream)
{
    IQ_CHECK_ARG(keys && values && k_strides && v_strides && pool && page_ids && flags && next_flags,
                 "iq_encode_pages: null pointer");
    IQ_CHECK_ARG(dtype == IQ_BF16 || dtype == IQ_F16, "iq_encode_pages: keys/values must be bf16 or f16");
    IQ_CHECK_ARG(id_bytes == 4 || id_bytes == 8, "iq_encode_pages: id_bytes");
    const int64_t B = block_tokens;
    IQ_CHECK_ARG(B == 16 || B == 32 || B == 64 || B == 128 || B == 256, "iq_encode_pages: %lld-token pages",
                 (long long)B);
    IQ_CHECK_ARG(n_pages >= 0 && n_pages <= 0x7fffffffLL && H >= 1 && H <= 65535, "iq_encode_pages: shape");
    // rows read as 16-byte vectors (keys through direct-to-LDS chunk loads)
    auto rows_ok = [](const void *p, const int64_t *st) {
        return ((uintptr_t)p & 15) == 0 && st[3] == 1 && st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0 &&
               st[2] >= 0 && st[2] <= (1 << 24);
    };
    IQ_CHECK_ARG(rows_ok(keys, k_strides) && rows_ok(values, v_strides),
                 "iq_encode_pages: key/value rows must be contiguous and 16-byte aligned");
    const int64_t page_bytes = H * (104 * B + 832);
    K4Args a{};
    a.x = keys;
    a.dt = dtype;
    a.sb = k_strides[0];
    a.sh = k_strides[1];
    a.st = k_strides[2];
    a.sc = 1;
    a.H = H;
    a.T = B;
    a.D = TILE_D;
    a.count = 16;
    a.stride = 8;
    a.min_error = 1;
    a.bad = flags;
    a.pool = pool;
    a.pool_pages = pool_pages;
    a.page_bytes = page_bytes;
    a.ids = page_ids;
    a.id_bytes = id_bytes;
    a.off_kpay = 0;
    a.off_kscale = H * B * 64;
    a.off_kmap = a.off_kscale + H * 128 * 4;
    a.off_kpad = a.off_kmap + H * 128 * 2;
    a.off_vpay = a.off_kpad + H * 16 * 4;
    a.off_vscale = a.off_vpay + H * B * 32;
    a.off_voff = a.off_vscale + H * B * 2 * 2;
    a.v = (const uint16_t *)values;
    a.vsb = v_strides[0];
    a.vsh = v_strides[1];
    a.vst = v_strides[2];
    a.vbad = flags + 1;
    a.badid = flags + 2;
    a.clear = next_flags;
    a.page_rows = page_rows;
    if (n_pages == 0) return IQ_OK;
    const hipStream_t st = (hipStream_t)stream;
    if (B <= 32) {
        // one wavefront per (page, head) row, four pages of one head per workgroup
        const dim3 rows_grid((unsigned)((n_pages + 3) / 4), (unsigned)H);
        if (dtype == IQ_F16) {
            if (B == 16) hipLaunchKernelGGL((k4_encode_page_rows<true, 16>), rows_grid, dim3(K4_THREADS), 0, st, a, n_pages);
            else hipLaunchKernelGGL((k4_encode_page_rows<true, 32>), rows_grid, dim3(K4_THREADS), 0, st, a, n_pages);
        } else {
            if (B == 16) hipLaunchKernelGGL((k4_encode_page_rows<false, 16>), rows_grid, dim3(K4_THREADS), 0, st, a, n_pages);
            else hipLaunchKernelGGL((k4_encode_page_rows<false, 32>), rows_grid, dim3(K4_THREADS), 0, st, a, n_pages);
        }
        IQ_CHECK_LAUNCH("k4_encode_page_rows");
        return IQ_OK;
    }
    const dim3 grid((unsigned)n_pages, (unsigned)H), block(K4_THREADS);
    if (dtype == IQ_F16) {
        if (B == TILE_T) hipLaunchKernelGGL((k4_encode_tile<true, TILE_T / CH, true>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((k4_encode_tile<true, 0, true>), grid, block, 0, st, a);
    } else {
        if (B == TILE_T) hipLaunchKernelGGL((k4_encode_tile<false, TILE_T / CH, true>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((k4_encode_tile<false, 0, true>), grid, block, 0, st, a);
    }
    IQ_CHECK_LAUNCH("k4_encode_tile (pages)");
    return IQ_OK;
}
