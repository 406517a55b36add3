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

// Lanes' versions of iq_bit_below / iq_bit_above for D = 128 (two mask words,
// per-lane position).
__device__ __forceinline__ int iq_lane_bit_below(uint64_t m0, uint64_t m1, int pos)
{
    const uint64_t w1 = pos <= 64 ? 0ull : pos >= 128 ? m1 : m1 & ((1ull << (pos - 64)) - 1);
    const uint64_t w0 = pos <= 0 ? 0ull : pos >= 64 ? m0 : m0 & ((1ull << pos) - 1);
    return w1 ? 127 - __builtin_clzll(w1) : w0 ? 63 - __builtin_clzll(w0) : -1;
}

__device__ __forceinline__ int iq_lane_bit_above(uint64_t m0, uint64_t m1, int pos)
{
    const uint64_t w0 = pos >= 63 ? 0ull : pos < 0 ? m0 : m0 & ~((2ull << pos) - 1);
    const uint64_t w1 = pos >= 127 ? 0ull : pos < 64 ? m1 : m1 & ~((2ull << (pos - 64)) - 1);
    return w0 ? __builtin_ctzll(w0) : w1 ? 64 + __builtin_ctzll(w1) : 128;
}

// The sequential donor picks of iq_select_wave_t<2> for one D = 128 row, run
// by one wavefront: sel0 / sel1 mark the sources (channels lane and
// 64 + lane), av0 / av1 the channels that may donate.  The neighbour order
// and run boundaries are precomputed one source per lane, so a pick with a
// free neighbour is a handful of scalar operations.  LDS scratch: list[64].
__device__ __forceinline__ void iq_pick_donors128(const float *sal, uint64_t sel0, uint64_t sel1, uint64_t av0,
                                                  uint64_t av1, int count, int16_t *src_out, int16_t *don_out,
                                                  uint8_t *is_src, int16_t *src_of, int16_t *list)
{
    const int lane = threadIdx.x & 63;
    const uint64_t below = (1ull << lane) - 1;
    if ((sel0 >> lane) & 1ull) list[__popcll(sel0 & below)] = (int16_t)lane;
    if ((sel1 >> lane) & 1ull) list[__popcll(sel0) + __popcll(sel1 & below)] = (int16_t)(64 + lane);
    // lanes read list entries other lanes of this wavefront wrote: LDS
    // operations of a wavefront complete in order, so this fence emits
    // nothing; it keeps the compiler from moving the reads above the writes
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    is_src[lane] = (uint8_t)((sel0 >> lane) & 1ull);
    is_src[64 + lane] = (uint8_t)((sel1 >> lane) & 1ull);
    src_of[lane] = -1;
    src_of[64 + lane] = -1;
    const uint32_t sk0 = iq_nonneg_bits(sal[lane]), sk1 = iq_nonneg_bits(sal[64 + lane]);
    // lane i: the i-th source s, whether its left neighbour wins a saliency
    // comparison with the right one, and its selected run [lb, rb], packed
    // into one word so that a pick reads them with a single readlane
    const int s = lane < count ? list[lane] : 0;
    const uint32_t kl = s >= 1 ? iq_nonneg_bits(sal[s - 1]) : ~0u;
    const uint32_t kr = s + 1 < 128 ? iq_nonneg_bits(sal[s + 1]) : ~0u;
    const int lb = iq_lane_bit_below(~sel0, ~sel1, s) + 1;
    const int rb = iq_lane_bit_above(~sel0, ~sel1, s) - 1;
    const uint32_t wv = (uint32_t)s | ((kl <= kr ? 1u : 0u) << 8) | ((uint32_t)lb << 9) | ((uint32_t)(rb + 1) << 17);
    int don_v = 0;
    for (int i = 0; i < count; ++i) {
        const uint32_t w = __builtin_amdgcn_readlane(wv, i);
        const int si = (int)(w & 255u), l1 = si - 1, r1 = si + 1;
        const bool lo = l1 >= 0 && (((l1 < 64 ? av0 : av1) >> (l1 & 63)) & 1ull);
        const bool ro = r1 < 128 && (((r1 < 64 ? av0 : av1) >> (r1 & 63)) & 1ull);
        int donor;
        if (lo || ro) {
            donor = (lo && (!ro || ((w >> 8) & 1u))) ? l1 : r1;
        } else {
            // the nearest available channel below the run or above it; less
            // saliency, then the lower channel, on a distance tie
            const int lbi = (int)((w >> 9) & 255u), rbi = (int)((w >> 17) & 255u) - 1;
            const uint64_t m[2] = {av0, av1};
            const int pl = iq_bit_below<2>(m, lbi);
            const int pr = iq_bit_above<2>(m, rbi, 128);
            const int dl = pl >= 0 ? lbi - pl : 0x7fffffff;
            const int dr = pr < 128 ? pr - rbi : 0x7fffffff;
            donor = 0;            // an empty pool only arises from non-finite statistics
            if (dl < dr) donor = pl;
            else if (dr < dl) donor = pr;
            else if (dl != 0x7fffffff) {
                const uint32_t ka = __builtin_amdgcn_readlane(pl < 64 ? sk0 : sk1, pl & 63);
                const uint32_t kb = __builtin_amdgcn_readlane(pr < 64 ? sk0 : sk1, pr & 63);
                donor = ka <= kb ? pl : pr;
            }
        }
        if (donor < 64) av0 &= ~(1ull << donor);
        else av1 &= ~(1ull << (donor - 64));
        don_v = lane == i ? donor : don_v;
    }
    if (lane < count) {
        src_out[lane] = (int16_t)s;
        don_out[lane] = (int16_t)don_v;
        src_of[don_v] = (int16_t)s;
    }
}

// The selection of iq_select_wave_t<2> for one D = 128 row, computed by a
// whole 256-thread workgroup (every thread calls it: it holds barriers).
// Sources and the min_error pool come from ranks over all channel pairs:
// each channel gets a 64-bit key that orders it exactly as the stable sort
// does (the value's bits, then the channel as tie-break), and its rank is the
// number of keys ordered before it, each thread comparing against 64 of
// them.  The sequential donor picks then run on one wavefront (threads 0-63 of the order the caller passes) from the neighbour
// order and run boundaries precomputed one source per lane, so a pick with a
// free neighbour is a handful of scalar operations.  LDS scratch: key[128],
// part[256], flag[128], list[64].
__device__ __forceinline__ void iq_select_tile128(const float *sal, const float *err, int count,
                                                  int16_t *src_out, int16_t *don_out, uint8_t *is_src,
                                                  int16_t *src_of, uint64_t *key, int *part, uint8_t *flag,
                                                  int16_t *list, int tid)
{
    typedef __attribute__((ext_vector_type(2))) uint64_t v2u64;
    const int c = tid & 127, half = tid >> 7, lane = tid & 63;
    // 1. sources: the `count` channels first in descending saliency, ties to
    //    the lower channel; as one ascending key: ~bits, then the channel
    if (tid < 128) key[c] = ((uint64_t)~iq_nonneg_bits(sal[c]) << 7) | (uint64_t)c;
    __syncthreads();
    {
        const uint64_t mine = key[c];
        int r = 0;
#pragma unroll 8
        for (int k = 0; k < 64; k += 2) {
            const v2u64 kk = *(const v2u64 *)(key + 64 * half + k);
            r += kk[0] < mine;
            r += kk[1] < mine;
        }
        part[tid] = r;
    }
    __syncthreads();
    const bool sel = part[c] + part[c + 128] < count;
    bool avail = !sel;
    if (err) {  // 2. pool: the `count` non-sources first in ascending error, ties to the lower channel
        if (tid < 128) key[c] = sel ? ~0ull : ((uint64_t)iq_nonneg_bits(err[c]) << 7) | (uint64_t)c;
        __syncthreads();
        const uint64_t mine = key[c];
        int r = 0;
#pragma unroll 8
        for (int k = 0; k < 64; k += 2) {
            const v2u64 kk = *(const v2u64 *)(key + 64 * half + k);
            r += kk[0] < mine;
            r += kk[1] < mine;
        }
        __syncthreads();            // every thread has read part[] for sel
        part[tid] = r;
        __syncthreads();
        avail = !sel && part[c] + part[c + 128] < count;
    }
    if (tid < 128) flag[c] = (sel ? 1 : 0) | (avail ? 2 : 0);
    __syncthreads();
    if (tid >= 64) return;

    // 3. sequential donor picks on the wavefront of tid 0-63; sources in ascending channel order
    const uint32_t f0 = flag[lane], f1 = flag[64 + lane];
    iq_pick_donors128(sal, __ballot(f0 & 1u), __ballot(f1 & 1u), __ballot(f0 & 2u), __ballot(f1 & 2u), count, src_out,
                      don_out, is_src, src_of, list);
}

// Top `count` of the 128 keys k0 (channel lane) and k1 (channel 64 + lane)
// among the eligible channels (masks e0, e1), ties to the lower channel: the
// selection of iq_wave_top<2>, with the comparisons made straight into lane
// masks.  Ineligible keys are zeroed first, so that the radix search, whose
// candidates are never 0, needs no mask; only the ties at the threshold do.
__device__ __forceinline__ void iq_top128(uint32_t k0, uint32_t k1, uint64_t e0, uint64_t e1, int count, uint64_t &o0,
                                          uint64_t &o1)
{
    constexpr int UGT = 34, UGE = 35, EQ = 32;    // integer predicates of the lane-mask compares
    const int lane = threadIdx.x & 63;
    k0 = ((e0 >> lane) & 1ull) ? k0 : 0u;
    k1 = ((e1 >> lane) & 1ull) ? k1 : 0u;
    if (count <= 0) {
        o0 = o1 = 0;
        return;
    }
    uint32_t thr = 0;
#pragma unroll
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = thr | (1u << bit);
        const int n = __popcll(__builtin_amdgcn_uicmp(k0, cand, UGE)) + __popcll(__builtin_amdgcn_uicmp(k1, cand, UGE));
        if (n >= count) thr = cand;
    }
    o0 = __builtin_amdgcn_uicmp(k0, thr, UGT) & e0;
    o1 = __builtin_amdgcn_uicmp(k1, thr, UGT) & e1;
    int need = count - __popcll(o0) - __popcll(o1);
    uint64_t eq0 = __builtin_amdgcn_uicmp(k0, thr, EQ) & e0, eq1 = __builtin_amdgcn_uicmp(k1, thr, EQ) & e1;
    for (; eq0 && need > 0; --need) {
        const uint64_t low = eq0 & (~eq0 + 1);
        o0 |= low;
        eq0 ^= low;
    }
    for (; eq1 && need > 0; --need) {
        const uint64_t low = eq1 & (~eq1 + 1);
        o1 |= low;
        eq1 ^= low;
    }
}

// The selection of iq_select_wave_t<2> for one D = 128 row by one wavefront
// (sal / err in LDS, err null for the plain policy): radix top-k for the
// sources and the min_error pool, then iq_pick_donors128.  LDS scratch:
// list[64].
__device__ __forceinline__ void iq_select_wave128(const float *sal, const float *err, int count, int16_t *src_out,
                                                  int16_t *don_out, uint8_t *is_src, int16_t *src_of, int16_t *list)
{
    const int lane = threadIdx.x & 63;
    uint64_t sel0, sel1;
    iq_top128(iq_nonneg_bits(sal[lane]), iq_nonneg_bits(sal[64 + lane]), ~0ull, ~0ull, count, sel0, sel1);
    uint64_t av0 = ~sel0, av1 = ~sel1;
    if (err)  // ascending error == descending complement of its bit pattern
        iq_top128(~iq_nonneg_bits(err[lane]), ~iq_nonneg_bits(err[64 + lane]), ~sel0, ~sel1, count, av0, av1);
    iq_pick_donors128(sal, sel0, sel1, av0, av1, count, src_out, don_out, is_src, src_of, list);
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
