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

__device__ __forceinline__ uint64_t iq_wave_min_u64(uint64_t v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        uint64_t o = __shfl_xor(v, off, 64);
        v = o < v ? o : v;
    }
    return v;
}

__device__ __forceinline__ int iq_wave_max_i32(int v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ int iq_wave_min_i32(int v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = min(v, __shfl_xor(v, off, 64));
    return v;
}

// Total order used by torch's stable sorts on non-NaN floats, as integers.
__device__ __forceinline__ uint32_t iq_nonneg_bits(float f) { return __float_as_uint(f); }

// sal/err: LDS arrays of D floats (err may be null).  Outputs src/don
// (count entries each, LDS) and is_src / src_of (LDS, D entries) describing
// roles for the quantizer.  Must be called by exactly one full wavefront.
__device__ void iq_select_wave(const float *sal, const float *err, int D, int count,
                               int16_t *src_out, int16_t *don_out, uint8_t *is_src, int16_t *src_of)
{
    const int lane = threadIdx.x & 63;
    const int nchunk = (D + 63) / 64;
    uint64_t sel_mask[IQ_MAXCHUNK];
    uint64_t avail_mask[IQ_MAXCHUNK];

    // 1. stable top-`count` by saliency
    for (int k = 0; k < nchunk; ++k) {
        const int c = k * 64 + lane;
        bool selected = false;
        if (c < D) {
            const float sc = sal[c];
            int rank = 0;
            for (int o = 0; o < D; ++o) {
                const float so = sal[o];
                rank += (so > sc) || (so == sc && o < c);
            }
            selected = rank < count;
        }
        sel_mask[k] = __ballot(selected);
    }
    // 2. donor pool
    for (int k = 0; k < nchunk; ++k) {
        const int c = k * 64 + lane;
        bool avail = false;
        if (c < D) {
            const bool selected = (sel_mask[k] >> lane) & 1ull;
            if (err) {
                const float inf = __uint_as_float(0x7f800000u);
                const float ec = selected ? inf : err[c];
                int rank = 0;
                for (int o = 0; o < D; ++o) {
                    const bool so_sel = (sel_mask[o >> 6] >> (o & 63)) & 1ull;
                    const float eo = so_sel ? inf : err[o];
                    rank += (eo < ec) || (eo == ec && o < c);
                }
                avail = rank < count;
            } else {
                avail = !selected;
            }
        }
        avail_mask[k] = __ballot(avail);
    }
    // role tables for the quantizer (filled in as sources are assigned)
    for (int c = lane; c < D; c += 64) {
        is_src[c] = 0;
        src_of[c] = -1;
    }

    // 3. sequential donor picks; sources visited in ascending channel order
    int i = 0;
    for (int k = 0; k < nchunk; ++k) {
        uint64_t m = sel_mask[k];
        while (m && i < count) {
            const int bit = __builtin_ctzll(m);
            m &= m - 1;
            const int s = k * 64 + bit;
            const bool left_ok = s - 1 >= 0 && ((avail_mask[(s - 1) >> 6] >> ((s - 1) & 63)) & 1ull);
            const bool right_ok = s + 1 < D && ((avail_mask[(s + 1) >> 6] >> ((s + 1) & 63)) & 1ull);
            uint64_t best = ~0ull;
            if (left_ok || right_ok) {
                for (int kk = 0; kk < nchunk; ++kk) {
                    const int p = kk * 64 + lane;
                    const bool cand = (p == s - 1 && left_ok) || (p == s + 1 && right_ok);
                    if (cand) {
                        const uint64_t key = ((uint64_t)iq_nonneg_bits(sal[p]) << 11) | (uint64_t)p;
                        best = key < best ? key : best;
                    }
                }
            } else {
                // boundaries of the contiguous salient run containing s
                int left = -1, right = D;
                for (int kk = 0; kk < nchunk; ++kk) {
                    const int p = kk * 64 + lane;
                    const bool nonsel = p < D && !((sel_mask[kk] >> lane) & 1ull);
                    if (nonsel && p < s) left = max(left, p);
                    if (nonsel && p > s) right = min(right, p);
                }
                left = iq_wave_max_i32(left) + 1;
                right = iq_wave_min_i32(right) - 1;
                for (int kk = 0; kk < nchunk; ++kk) {
                    const int p = kk * 64 + lane;
                    if (p < D && ((avail_mask[kk] >> lane) & 1ull)) {
                        const int dl = abs(p - left), dr = abs(p - right);
                        const uint64_t dist = (uint64_t)min(dl, dr);
                        const uint64_t key = (dist << 43) | ((uint64_t)iq_nonneg_bits(sal[p]) << 11) | (uint64_t)p;
                        best = key < best ? key : best;
                    }
                }
            }
            best = iq_wave_min_u64(best);
            // An empty candidate set only arises from non-finite statistics,
            // whose outputs the caller discards; stay in bounds regardless.
            const int donor = best == ~0ull ? 0 : (int)(best & 2047ull);
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
