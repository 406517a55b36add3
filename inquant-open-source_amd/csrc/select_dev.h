// Wave-level donor selection (one 64-lane wavefront per row).
//
// Restates the reference's two selectors, which agree by construction:
// codec.py:137-178 (_reuse_map, torch) and triton_selection.py:11-43 (_select).
//   1. sources = the `count` channels of largest saliency, ties to the lower
//      channel (stable descending argsort), listed in ascending order;
//   2. min_error: only the `count` non-source channels of smallest donor
//      error (ties to the lower channel) may donate; otherwise every
//      non-source channel may;
//   3. for each source s in ascending order: candidates are the available
//      immediate neighbours s-1, s+1; if none, the available channels at the
//      smallest distance from either boundary of s's contiguous salient run;
//      the donor is the candidate of least saliency, lowest channel on ties.
// Saliency and error are non-negative, so their IEEE bit patterns order them.
#pragma once

#include "iq_common.h"

#define IQ_MAXD 1024
#define IQ_MAXCHUNK (IQ_MAXD / 64)

// Total order used by torch's stable sorts on non-NaN floats, as integers.
__device__ __forceinline__ uint32_t iq_nonneg_bits(float f) { return __float_as_uint(f); }

// Marks in out[] the `count` eligible lanes of largest key, ties to the lower
// channel (channel = 64 k + lane), which is the stable descending sort's
// top `count`.  The count-th largest key is found by a bitwise radix search
// over ballots, then ties at that key are taken in channel order.
template <int NC>
__device__ __forceinline__ void iq_wave_top(const uint32_t (&key)[NC], const uint64_t (&elig)[NC], int count,
                                            uint64_t (&out)[NC])
{
    const int lane = threadIdx.x & 63;
    if (count <= 0) {
#pragma unroll
        for (int k = 0; k < NC; ++k) out[k] = 0;
        return;
    }
    uint32_t thr = 0;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = thr | (1u << bit);
        int n = 0;
#pragma unroll
        for (int k = 0; k < NC; ++k)
            n += __popcll(__ballot(((elig[k] >> lane) & 1ull) && key[k] >= cand));
        if (n >= count) thr = cand;
    }
    int need = count;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        out[k] = __ballot(((elig[k] >> lane) & 1ull) && key[k] > thr);
        need -= __popcll(out[k]);
    }
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        uint64_t eq = __ballot(((elig[k] >> lane) & 1ull) && key[k] == thr);
        while (eq && need > 0) {
            const uint64_t low = eq & (~eq + 1);
            out[k] |= low;
            eq ^= low;
            --need;
        }
    }
}

// key[c >> 6] of lane c & 63 (c wave-uniform), read without a cross-lane exchange.
template <int NC>
__device__ __forceinline__ uint32_t lane_key(const uint32_t (&key)[NC], int c)
{
    uint32_t v = 0;
#pragma unroll
    for (int k = 0; k < NC; ++k)
        if ((c >> 6) == k) v = __builtin_amdgcn_readlane(key[k], c & 63);
    return v;
}

// Highest set bit of the NC-word mask strictly below pos, or -1.
template <int NC>
__device__ __forceinline__ int iq_bit_below(const uint64_t (&m)[NC], int pos)
{
    int r = -1;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        const int base = 64 * k;
        uint64_t w = pos <= base ? 0ull : pos >= base + 64 ? m[k] : m[k] & ((1ull << (pos - base)) - 1);
        if (w) r = base + 63 - __builtin_clzll(w);
    }
    return r;
}

// Lowest set bit of the NC-word mask strictly above pos, or `none`.
template <int NC>
__device__ __forceinline__ int iq_bit_above(const uint64_t (&m)[NC], int pos, int none)
{
    int r = none;
#pragma unroll
    for (int k = NC - 1; k >= 0; --k) {
        const int base = 64 * k;
        uint64_t w = pos >= base + 63 ? 0ull : pos < base ? m[k] : m[k] & ~((2ull << (pos - base)) - 1);
        if (w) r = base + __builtin_ctzll(w);
    }
    return r;
}

// sal/err: LDS arrays of D floats (err may be null), D <= 64 * NC.  Outputs
// src/don (count entries each, LDS) and is_src / src_of (LDS, D entries)
// describing roles for the quantizer.  Must be called by exactly one full
// wavefront.  Saliencies and errors stay in registers as their bit patterns.
template <int NC>
__device__ __forceinline__ void iq_select_wave_t(const float *sal, const float *err, int D, int count,
                                 int16_t *src_out, int16_t *don_out, uint8_t *is_src, int16_t *src_of)
{
    const int lane = threadIdx.x & 63;
    uint32_t skey[NC], ekey[NC];
    uint64_t valid[NC], sel_mask[NC], avail_mask[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        const int c = k * 64 + lane;
        const bool ok = c < D;
        skey[k] = ok ? iq_nonneg_bits(sal[c]) : 0u;
        // ascending error == descending complement of its bit pattern
        ekey[k] = ok && err ? ~iq_nonneg_bits(err[c]) : 0u;
        valid[k] = __ballot(ok);
    }
    // 1. stable top-`count` by saliency
    iq_wave_top<NC>(skey, valid, count, sel_mask);
    // 2. donor pool: every other channel, or the `count` of least error
    uint64_t rest[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) rest[k] = valid[k] & ~sel_mask[k];
    if (err) iq_wave_top<NC>(ekey, rest, count, avail_mask);
    else
#pragma unroll
        for (int k = 0; k < NC; ++k) avail_mask[k] = rest[k];
    uint64_t nonsel[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) nonsel[k] = valid[k] & ~sel_mask[k];
    // role tables for the quantizer (filled in as sources are assigned)
    for (int c = lane; c < D; c += 64) {
        is_src[c] = 0;
        src_of[c] = -1;
    }

    // 3. sequential donor picks; sources visited in ascending channel order
    int i = 0;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        uint64_t m = sel_mask[k];
        while (m && i < count) {
            const int bit = __builtin_ctzll(m);
            m &= m - 1;
            const int s = k * 64 + bit;
            const bool left_ok = s - 1 >= 0 && ((avail_mask[(s - 1) >> 6] >> ((s - 1) & 63)) & 1ull);
            const bool right_ok = s + 1 < D && ((avail_mask[(s + 1) >> 6] >> ((s + 1) & 63)) & 1ull);
            int donor = 0;            // an empty pool only arises from non-finite statistics
            if (left_ok || right_ok) {
                // at most two candidates: read their saliencies from their lanes
                // (lower saliency wins, the lower channel on ties)
                const uint32_t kl = left_ok ? lane_key<NC>(skey, s - 1) : ~0u;
                const uint32_t kr = right_ok ? lane_key<NC>(skey, s + 1) : ~0u;
                donor = (!right_ok || (left_ok && kl <= kr)) ? s - 1 : s + 1;
            } else {
                // The run of selected channels around s is [lb, rb]; every
                // available channel lies outside it, so the nearest available
                // channel to either boundary is the highest one below lb or the
                // lowest one above rb (less saliency, then lower channel, on a
                // distance tie).  Bit scans of the uniform masks find both.
                const int lb = iq_bit_below<NC>(nonsel, s) + 1;
                const int rb = iq_bit_above<NC>(nonsel, s, D) - 1;
                const int pl = iq_bit_below<NC>(avail_mask, lb);
                const int pr = iq_bit_above<NC>(avail_mask, rb, D);
                const int dl = pl >= 0 ? lb - pl : 0x7fffffff;
                const int dr = pr < D ? pr - rb : 0x7fffffff;
                if (dl < dr) donor = pl;
                else if (dr < dl) donor = pr;
                else if (dl != 0x7fffffff)
                    donor = lane_key<NC>(skey, pl) <= lane_key<NC>(skey, pr) ? pl : pr;
            }
            avail_mask[donor >> 6] &= ~(1ull << (donor & 63));
            if (lane == 0) {
                is_src[s] = 1;
                src_out[i] = (int16_t)s;
                don_out[i] = (int16_t)donor;
                src_of[donor] = (int16_t)s;
            }
            ++i;
        }
    }
}

__device__ __forceinline__ void iq_select_wave(const float *sal, const float *err, int D, int count,
                                               int16_t *src_out, int16_t *don_out, uint8_t *is_src,
                                               int16_t *src_of)
{
    if (D <= 64) iq_select_wave_t<1>(sal, err, D, count, src_out, don_out, is_src, src_of);
    else if (D <= 128) iq_select_wave_t<2>(sal, err, D, count, src_out, don_out, is_src, src_of);
    else if (D <= 256) iq_select_wave_t<4>(sal, err, D, count, src_out, don_out, is_src, src_of);
    else if (D <= 512) iq_select_wave_t<8>(sal, err, D, count, src_out, don_out, is_src, src_of);
    else iq_select_wave_t<16>(sal, err, D, count, src_out, don_out, is_src, src_of);
}
