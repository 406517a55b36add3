// Causal prefill attention over exact K/V on matrix cores (gfx950).
//
// Replaces the vLLM plugin's prefill call
//   flash_attn_varlen_func(q, k, v, out, cu_seqlens_q=cu, cu_seqlens_k=cu,
//                          max_seqlen_q=n, max_seqlen_k=n, causal=True, softmax_scale)
// (extensions/vllm/src/inquant_vllm/backend.py:139-144): every query attends to
// the keys at or before its position in its own sequence, in the K/V dtype
// with fp32 logits, softmax and accumulation.  Layout is vLLM's token-major
// [tokens, heads, 128] with runtime (token, head) strides; sequences are
// delimited by cu_seqlens.
//
// One workgroup = 128 queries of one query head: four wavefronts of 32
// queries, one per SIMD, so the two wavefronts that share a SIMD belong to
// different workgroups and overlap each other's matrix products with their
// softmax.  Keys are the rows of S^T = K Q^T on v_mfma_f32_32x32x16 (queries
// as columns): lane (query l % 32, half l / 32) holds 16 keys of its query per
// 32-key block, so the row maximum is an in-lane maximum and one permlane32
// swap, and the softmax weights land in the lanes and k-slots of the B
// operand of O^T = V^T P^T (k-slot 8 h + i of a 16-key chunk c is key
// 16 c + 4 h + i % 4 + 8 (i / 4)), so P needs no transpose.  Per 32 queries a
// key byte read from LDS feeds twice the products of 16-query wavefronts on
// 16x16x32 (0.92 -> 0.75 ms for the 8K causal Qwen2.5-7B prefill; earlier
// forms: 2.16 ms with four wavefronts of 16, 1.13 ms with eight and register
// double buffering, two 16-query subtiles per wavefront 1.33 ms).  Key tiles
// of 64 stream global -> LDS by direct loads (no registers) into two LDS
// stages of row-major K and V with XOR-swizzled 16-byte chunks; the V
// operand of O^T = V^T P^T comes out of LDS already transposed
// (ds_read_b64_tr_b16); one barrier per tile.  Masks only on the diagonal
// and last tiles; query tiles longest-first, each XCD on a contiguous range
// of (query head, tile) items.  184 VGPRs: two wavefronts per SIMD.
#include "decode_common.h"

namespace {

constexpr int D = 128;
constexpr int NW = 4;               // wavefronts per workgroup
constexpr int NT = 64 * NW;         // threads per workgroup
constexpr int QW = 32;              // queries per wavefront
constexpr int QT = QW * NW;         // queries per workgroup
constexpr int KT = 64;              // keys per tile

typedef __attribute__((ext_vector_type(16))) float f32x16;

struct PrefillArgs {
    const uint16_t *q, *k, *v;
    void *out;
    int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh;   // element strides (token, head)
    const int32_t *cu;                                        // [n_seq + 1] token offsets
    int tiles, Hq;                                            // query tiles per sequence, query heads
    int G;
    float c_log2;                                             // softmax scale * log2(e)
    int odt;
    int vec_out;                                              // output rows aligned for 4-channel stores
};

// two stages: one is computed while the next tile lands in the other.  Rows
// of 128 channels (256 bytes); the 16-byte chunk c of K row r sits at chunk
// slot c ^ (r % 16) and that of V row r at slot c ^ 4 (r % 4), so that the
// operand reads below hit 64 distinct banks per 16 (K) or 32 (V) lanes.
struct __attribute__((aligned(16))) PrefillSmem {
    uint16_t k[2][KT * D];
    uint16_t v[2][KT * D];
};
static_assert(2 * sizeof(PrefillSmem) <= 160 * 1024, "two workgroups per compute unit");

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element
// i % 4 of the 4 halves that lanes i / 4, i / 4 + 4, i / 4 + 8 and i / 4 + 12
// address (in that order).  When lane s reads key K0 + s / 4, channels
// c0 + 4 (s % 4) .. + 3, lane i receives channel c0 + i of keys K0 .. K0 + 3.
typedef short gv16x4 __attribute__((__vector_size__(4 * sizeof(short))));
__device__ __forceinline__ u32x2 tr_read(const uint16_t *p)
{
    const gv16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) gv16x4 *)(__attribute__((address_space(3))) uint16_t *)p);
    return __builtin_bit_cast(u32x2, v);
}

// 32x32x16 product: lane l holds A[l % 32][8 (l / 32) .. + 7], B[8 (l / 32) .. + 7][l % 32]
// and C[8 (i / 4) + 4 (l / 32) + i % 4][l % 32] in register i
template <bool F16>
__device__ __forceinline__ f32x16 mma3232(u32x4 a, u32x4 b, f32x16 c)
{
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
}

// reductions over the lane pair l, l ^ 32 (one query's two halves)
__device__ __forceinline__ float pair_max(float v)
{
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
}

__device__ __forceinline__ float pair_sum(float v)
{
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(h[0]) + __uint_as_float(h[1]);
}

template <bool F16>
__global__ __launch_bounds__(NT, 2) void prefill_attn(PrefillArgs a)
{
    __shared__ PrefillSmem sm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c32 = lane & 31, h32 = lane >> 5;
    // Workgroup i of a sequence's slice runs on XCD i % 8 (the dispatcher
    // deals workgroups round-robin over the eight XCDs; every slice is a
    // multiple of 8 long).  Each XCD takes a contiguous range of the slice's
    // (query head, query tile) items, so the workgroups resident on it read
    // the K/V of one or two KV heads and find them in its own L2 (8K causal
    // Qwen2.5-7B: 713 -> 577 us against items dealt out in grid order).
    // Within a query head, tiles go longest first.
    const int per = (a.tiles * a.Hq + 7) / 8;
    const int item = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (item >= a.tiles * a.Hq) return;          // the slice's padding
    const int hq = item / a.tiles, seq = blockIdx.y, h = hq / a.G;
    const int start = a.cu[seq], len = a.cu[seq + 1] - start;
    const int q0 = (a.tiles - 1 - item % a.tiles) * QT;
    if (q0 >= len) return;                       // uniform: no barrier is skipped by part of the group
    const int qw = q0 + QW * wave;               // this wavefront's first query
    const int my_q = qw + c32;                   // the query of this lane's column
    u32x4 qb[8];                                 // B operand: Q[my_q][16 d + 8 h32 .. + 7]
    {
        const int qq = my_q < len ? my_q : len - 1;
        const uint16_t *qp = a.q + (int64_t)(start + qq) * a.q_st + (int64_t)hq * a.q_sh + 8 * h32;
#pragma unroll
        for (int d = 0; d < 8; ++d) qb[d] = ld16(qp + 16 * d);
    }
    const uint16_t *kbase = a.k + (int64_t)start * a.k_st + (int64_t)h * a.k_sh;
    const uint16_t *vbase = a.v + (int64_t)start * a.v_st + (int64_t)h * a.v_sh;
    float m_run = NEG_INF, l_run = 0.0f;         // l_run: this lane's share of the column sum
    f32x16 acc[4];                               // O^T rows 32 db .. 32 db + 31 (output channels)
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[db][i] = 0.0f;
    const int kend = q0 + QT < len ? q0 + QT : len;
    // Key tiles stream global -> LDS directly (no registers).  Each wavefront
    // moves 16 of the tile's 64 rows of K and of V, four rows (1 KB) per
    // direct load: lane l fills chunk slot l % 16 of row l / 16 with the
    // chunk that belongs there under the swizzle.  Rows past the sequence's
    // end repeat its last row (masked).  Offsets are 32-bit from the tile's
    // first row (token strides below 2^25 elements).
    const uint32_t lds_k = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)&sm.k[0][0];
    const uint32_t lds_v = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)&sm.v[0][0];
    auto dma_tile = [&](int k0, int st) {
        const int last = len - 1 - k0;
        const uint16_t *kt = kbase + (int64_t)k0 * a.k_st, *vt = vbase + (int64_t)k0 * a.v_st;
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int r0 = 16 * wave + 4 * it;            // first row of this load (wave-uniform)
            const int r = r0 + (lane >> 4), p = lane & 15;
            const int rr = r < last ? r : last;
            const uint32_t ko = (uint32_t)((rr * a.k_st + 8 * (p ^ (r & 15))) * 2);
            const uint32_t vo = (uint32_t)((rr * a.v_st + 8 * (p ^ (4 * (r & 3)))) * 2);
            lds_load16(kt, ko, lds_k + (uint32_t)((st * KT + r0) * D * 2));
            lds_load16(vt, vo, lds_v + (uint32_t)((st * KT + r0) * D * 2));
        }
    };
    dma_tile(0, 0);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    int s = 0;
    for (int k0 = 0; k0 < kend; k0 += KT, s ^= 1) {
        // stage s ^ 1 was last read before the previous barrier
        if (k0 + KT < kend) dma_tile(k0 + KT, s ^ 1);
        if (k0 <= qw + QW - 1) {                 // some key of this tile is visible to this wavefront (uniform)
            const uint16_t *sk = sm.k[s];
            const uint16_t *sv = sm.v[s];
            // S^T blocks kb: lane holds keys k0 + 32 kb + 8 (i / 4) + 4 h32 + i % 4 of column my_q;
            // the two blocks' products alternate, so neither waits for its own previous one
            f32x16 sc[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) sc[kb][i] = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; ++d)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
                    sc[kb] = mma3232<F16>(*(const u32x4 *)(sk + (32 * kb + c32) * D + 8 * ((2 * d + h32) ^ (c32 & 15))),
                                          qb[d], sc[kb]);
            // raw logits: the scale is positive, so the maximum commutes with it
            // and p = 2^(s c - m) takes one fma per logit.  Only a tile that
            // reaches past this wavefront's first query or the sequence's end
            // has keys to mask (wave-uniform).
            if (k0 + KT - 1 > qw || k0 + KT > len) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int key = k0 + 32 * kb + 8 * (i >> 2) + 4 * h32 + (i & 3);
                        if (!(key <= my_q && key < len)) sc[kb][i] = NEG_INF;
                    }
            }
            float cmax = NEG_INF;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) cmax = fmaxf(cmax, sc[kb][i]);
            cmax = pair_max(cmax) * a.c_log2;
            // The reference maximum moves only when the tile's exceeds it by
            // more than 2^8 (or on the first tile): the weights 2^(s c - m) then
            // stay below 256, exact in range for the 16-bit P operand and the
            // fp32 sums, and the output rescale is skipped on most tiles.
            const float m_new = cmax > m_run + 8.0f ? cmax : m_run;   // finite: key 0 is visible to every query
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            float lsum = 0.0f;
            u32x4 pb[2][2];                          // B operand of the 16-key chunk (kb, c): registers 8 c .. 8 c + 7
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[kb][8 * c + 2 * w], a.c_log2, -m_new));
                        const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[kb][8 * c + 2 * w + 1], a.c_log2, -m_new));
                        lsum += p0;
                        lsum += p1;
                        pb[kb][c][w] = pack2<F16>(p0, p1);
                    }
            // the two lanes of a column share m, so their partial sums take
            // the same rescale and are added once, after the last tile
            l_run = fmaf(l_run, alpha, lsum);
            m_run = m_new;
            // alpha is exactly 1 wherever the maximum did not grow: when that
            // holds in every lane the rescale is the identity and is skipped
            if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
                for (int db = 0; db < 4; ++db) acc[db] *= alpha;
            }
            // A operand of chunk (kb, c): V^T row 32 db + c32, keys 32 kb + 16 c + 4 h32 + 0..3 and
            // + 8..11, as two transposed reads: lane s of a 16-lane group (g = the group's
            // half of the 32 rows) reads key K0 + s / 4, channels 32 db + 16 g + 4 (s % 4) .. + 3
            const int s16 = lane & 15, g = (lane >> 4) & 1;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int db = 0; db < 4; ++db) {
                        const int K0 = 32 * kb + 16 * c + 4 * h32 + (s16 >> 2);      // K0 % 4 == s16 / 4
                        const int cl = 4 * db + 2 * g + ((s16 & 3) >> 1);
                        const int sw = 4 * (s16 >> 2), half = 4 * (s16 & 1);
                        const u32x2 lo = tr_read(sv + K0 * D + 8 * (cl ^ sw) + half);
                        const u32x2 hi = tr_read(sv + (K0 + 8) * D + 8 * (cl ^ sw) + half);
                        acc[db] = mma3232<F16>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb[kb][c], acc[db]);
                    }
        }
        // this wavefront's direct loads of stage s ^ 1 have landed and its LDS
        // reads of stage s are done; after the barrier that holds for every
        // wavefront
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    l_run = pair_sum(l_run);
    if (my_q < len) {
        const float inv = 1.0f / l_run;
        const int64_t o = (int64_t)(start + my_q) * a.o_st + (int64_t)hq * a.o_sh + 4 * h32;
        // four consecutive channels per register group: one 16- or 8-byte store
        // when the rows are aligned for it (vec_out), else element by element
        if (a.vec_out && a.odt == IQ_F32) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    *(f32x4 *)((float *)a.out + o + 32 * db + 8 * g) =
                        f32x4{acc[db][4 * g] * inv, acc[db][4 * g + 1] * inv, acc[db][4 * g + 2] * inv,
                              acc[db][4 * g + 3] * inv};
        } else if (a.vec_out && a.odt != IQ_F32) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const bool f16 = a.odt == IQ_F16;
                    const float v0 = acc[db][4 * g] * inv, v1 = acc[db][4 * g + 1] * inv;
                    const float v2 = acc[db][4 * g + 2] * inv, v3 = acc[db][4 * g + 3] * inv;
                    *(u32x2 *)((uint16_t *)a.out + o + 32 * db + 8 * g) =
                        f16 ? u32x2{pack2<true>(v0, v1), pack2<true>(v2, v3)}
                            : u32x2{pack2<false>(v0, v1), pack2<false>(v2, v3)};
                }
        } else {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    iq_store_as(a.out, o + 32 * db + 8 * (i >> 2) + (i & 3), acc[db][i] * inv, a.odt);
        }
    }
}

}  // namespace

extern "C" int iq_prefill_attention(const void *q, const void *k, const void *v, int dtype, int64_t q_st,
                                    int64_t q_sh, int64_t k_st, int64_t k_sh, int64_t v_st, int64_t v_sh,
                                    const int32_t *cu_seqlens, int64_t n_seq, int64_t max_seqlen, int64_t Hq,
                                    int64_t H, int64_t head_dim, float scale, void *out, int64_t o_st,
                                    int64_t o_sh, int out_dtype, void *stream)
{
    IQ_CHECK_ARG(q && k && v && out && cu_seqlens, "iq_prefill_attention: null pointer");
    IQ_CHECK_ARG(dtype == IQ_BF16 || dtype == IQ_F16, "iq_prefill_attention: q/k/v must be bf16 or f16");
    IQ_CHECK_ARG(out_dtype >= IQ_F32 && out_dtype <= IQ_F16, "iq_prefill_attention: bad output dtype");
    IQ_CHECK_ARG(head_dim == D, "iq_prefill_attention: head_dim %lld (128 required)", (long long)head_dim);
    IQ_CHECK_ARG(H >= 1 && Hq >= 1 && Hq % H == 0 && Hq <= 65535, "iq_prefill_attention: heads %lld / %lld",
                 (long long)Hq, (long long)H);
    IQ_CHECK_ARG(n_seq >= 1 && n_seq <= 65535 && max_seqlen >= 1 && max_seqlen <= 0x7fffffffLL - QT,
                 "iq_prefill_attention: bad sequence count or length");
    // a key tile's rows are addressed by 32-bit byte offsets from its first row
    IQ_CHECK_ARG(k_st >= 0 && v_st >= 0 && k_st < (1LL << 25) && v_st < (1LL << 25),
                 "iq_prefill_attention: token stride too large");
    // rows are read as 16-byte vectors
    const uintptr_t bases = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v;
    IQ_CHECK_ARG(bases % 16 == 0 && (q_st | q_sh | k_st | k_sh | v_st | v_sh) % 8 == 0,
                 "iq_prefill_attention: q/k/v rows must be 16-byte aligned");
    // 4-channel output stores need every row start aligned to 4 elements' bytes
    const int64_t obytes = out_dtype == IQ_F32 ? 4 : 2;
    const int vec_out = (uintptr_t)out % (4 * obytes) == 0 && o_st % 4 == 0 && o_sh % 4 == 0;
    const int64_t tiles = (max_seqlen + QT - 1) / QT;
    // one slice of workgroups per sequence, padded to a multiple of 8
    const int64_t slice = (tiles * Hq + 7) / 8 * 8;
    IQ_CHECK_ARG(slice <= 0x7fffffffLL, "iq_prefill_attention: too many query tiles");
    PrefillArgs a{(const uint16_t *)q, (const uint16_t *)k, (const uint16_t *)v, out, q_st, q_sh, k_st, k_sh,
                  v_st, v_sh, o_st, o_sh, cu_seqlens, (int)tiles, (int)Hq, (int)(Hq / H),
                  scale * 1.44269504088896341f, out_dtype, vec_out};
    const dim3 grid((unsigned)slice, (unsigned)n_seq), block(NT);
    if (dtype == IQ_F16) hipLaunchKernelGGL(prefill_attn<true>, grid, block, 0, (hipStream_t)stream, a);
    else hipLaunchKernelGGL(prefill_attn<false>, grid, block, 0, (hipStream_t)stream, a);
    IQ_CHECK_LAUNCH("prefill_attn");
    return IQ_OK;
}
