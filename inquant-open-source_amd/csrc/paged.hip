// Paged packed-KV cache in the vLLM plugin's page layout (gfx950).
//
// Page format (extensions/vllm/src/inquant_vllm/layout.py:8-53), field-major
// within one page of H * (104 B + 832) bytes, B tokens per page, D = 128:
//   key_payload u8 [H, B, 64] | key_scales f32 [H, 128] | key_map i16 [H, 128]
//   | key_padding f32 [H, 16] | value_payload u8 [H, B, 32]
//   | value_scales f16 [H, B, 2] | value_offsets f16 [H, B, 2]
// key_map: -1 normal, the donor channel for a source, -2 - j for donor j.
//
// Kernels:
//   write_pages_kernel   codec outputs -> physical pages by id
//                        (packing.py:7-55 and the role map of layout.py:66-81)
//   unpack_pages_kernel  pages -> dense K/V of any dtype (layout.py:84-100)
//   decode_paged         fused single-query decode over a block table,
//                        batched over sequences (kernels.py:8-88)
//   paged_reduce         log-sum-exp merge of the per-partition partials
//
// decode_paged follows decode_fast: every load of a workgroup is issued up
// front, Q.K runs on matrix cores with the K tile decoded exactly in
// registers, salient codes are gathered into an extra 16x16x16 MFMA, the
// online softmax runs in the log2 domain and P.V uses hi + lo weights.  Pages
// shorter than a partition get their own per-channel constants, resolved
// from each page's role map as the reference decodes it: salient sources
// decode to zero in the 4-bit pass and take their 8-bit codes from the
// salient product, and a donor decodes to its padding through its constant
// pair.
#include "decode_common.h"

namespace {

constexpr int D = 128;
constexpr int WAVES = 4;
constexpr int PART = 256;              // tokens per partition
constexpr int VR = 132;                // dwords per staged token-pair row of decoded V (pairs t, t + 16)
constexpr int SELROW = D + 16;         // bytes per selection-matrix row (+16: the 16 rows of a read hit distinct banks)
constexpr int OROW = 132;              // floats per staged output row in the combine (conflict-free 16-byte stores)
constexpr int QROW = D + 8;            // u16 per staged query row (+8: rows of one column spread over the banks)
constexpr int SPG = 16;                // salient channels per page (the layout's key_padding width)
constexpr float LN2 = 0.693147180559945309f;

struct PageOffsets {
    int64_t ks, km, kp, vp, vs, vo;    // byte offsets of the fields after key_payload
};

__host__ __device__ inline PageOffsets page_offsets(int64_t H, int64_t B)
{
    PageOffsets o;
    o.ks = H * B * 64;
    o.km = o.ks + H * D * 4;
    o.kp = o.km + H * D * 2;
    o.vp = o.kp + H * SPG * 4;
    o.vs = o.vp + H * B * 32;
    o.vo = o.vs + H * B * 4;
    return o;
}

__device__ __forceinline__ int load_index(const void *p, int64_t i, int bytes)
{
    if (bytes == 1) return ((const uint8_t *)p)[i];
    if (bytes == 4) return ((const int32_t *)p)[i];
    return (int)((const int64_t *)p)[i];
}

__device__ __forceinline__ int64_t load_id(const void *p, int64_t i, int bytes)
{
    return bytes == 4 ? (int64_t)((const int32_t *)p)[i] : ((const int64_t *)p)[i];
}

// ------------------------------------------------------------------ writer

struct WriteArgs {
    const uint8_t *kp;                 // [n, H, B, 64]
    const float *ks;                   // [n, H, 128]
    const float *kpad;                 // [n, H, 16]
    const void *src, *don;             // [n, H, 16]
    int desc_bytes;
    const uint8_t *vp;                 // [n, H, B, 32]
    const uint16_t *vs, *vo;           // [n, H, B, 2]
    int64_t H, B, page_bytes, pool_pages;
    uint8_t *pool;
    const void *ids;
    int id_bytes;
    PageOffsets off;
};

// grid (n, H): one workgroup copies one (page, head) slice with 16-byte
// stores and builds its role map.  Ids outside the pool are skipped.
__global__ __launch_bounds__(256) void write_pages_kernel(WriteArgs a)
{
    __shared__ int16_t s_role[D];
    const int64_t n = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x;
    const int64_t id = load_id(a.ids, n, a.id_bytes);
    if (id < 0 || id >= a.pool_pages) return;
    uint8_t *page = a.pool + id * a.page_bytes;
    const int64_t nh = n * a.H + h;
    typedef __attribute__((ext_vector_type(4))) uint32_t v4;
    const v4 *ksrc = (const v4 *)(a.kp + nh * a.B * 64);
    v4 *kdst = (v4 *)(page + h * a.B * 64);
    for (int64_t i = tid; i < a.B * 4; i += 256) kdst[i] = ksrc[i];
    const v4 *vsrc = (const v4 *)(a.vp + nh * a.B * 32);
    v4 *vdst = (v4 *)(page + a.off.vp + h * a.B * 32);
    for (int64_t i = tid; i < a.B * 2; i += 256) vdst[i] = vsrc[i];
    uint16_t *vs = (uint16_t *)(page + a.off.vs) + h * a.B * 2;
    uint16_t *vo = (uint16_t *)(page + a.off.vo) + h * a.B * 2;
    for (int64_t i = tid; i < a.B * 2; i += 256) {
        vs[i] = a.vs[nh * a.B * 2 + i];
        vo[i] = a.vo[nh * a.B * 2 + i];
    }
    if (tid < D) {
        ((float *)(page + a.off.ks))[h * D + tid] = a.ks[nh * D + tid];
        s_role[tid] = -1;
    }
    if (tid < SPG) ((float *)(page + a.off.kp))[h * SPG + tid] = a.kpad[nh * SPG + tid];
    __syncthreads();
    if (tid < SPG) {
        const int s = load_index(a.src, nh * SPG + tid, a.desc_bytes);
        const int d = load_index(a.don, nh * SPG + tid, a.desc_bytes);
        if (s >= 0 && s < D) s_role[s] = (int16_t)d;
    }
    __syncthreads();
    if (tid < SPG) {
        const int d = load_index(a.don, nh * SPG + tid, a.desc_bytes);
        if (d >= 0 && d < D) s_role[d] = (int16_t)(-2 - tid);
    }
    __syncthreads();
    if (tid < D) ((int16_t *)(page + a.off.km))[h * D + tid] = s_role[tid];
}

// Pages of B = 16, 32 or 64 tokens: each 16-lane group writes one (page,
// head) slice with 16-byte copies, and builds its role map without LDS or
// barriers: lane j holds descriptor j and writes the roles of channels
// 8 j .. 8 j + 7, taking every descriptor from its lane of the group (all
// sources first, then all donors, as write_pages_kernel orders them).
template <int B>
__global__ __launch_bounds__(256) void write_small_pages_kernel(WriteArgs a, int64_t nph)
{
    typedef __attribute__((ext_vector_type(4))) uint32_t v4;
    const int tid = threadIdx.x, lane = tid & 63, j = tid & 15, g0 = lane & ~15;
    const int64_t ph = (int64_t)blockIdx.x * 16 + (tid >> 4);
    const int64_t nh = ph < nph ? ph : nph - 1;                       // clamped: every load valid
    const int64_t n = nh / a.H, h = nh % a.H;
    const int64_t id = load_id(a.ids, n, a.id_bytes);
    const bool live = ph < nph && id >= 0 && id < a.pool_pages;       // group-uniform
    const int s_j = load_index(a.src, nh * SPG + j, a.desc_bytes);
    const int d_j = load_index(a.don, nh * SPG + j, a.desc_bytes);
    int role[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) role[e] = -1;
#pragma unroll
    for (int k = 0; k < SPG; ++k) {
        const int sk = __builtin_amdgcn_ds_bpermute(4 * (g0 + k), s_j);
        const int dk = __builtin_amdgcn_ds_bpermute(4 * (g0 + k), d_j);
#pragma unroll
        for (int e = 0; e < 8; ++e) role[e] = sk >= 0 && sk < D && sk == 8 * j + e ? dk : role[e];
    }
#pragma unroll
    for (int k = 0; k < SPG; ++k) {
        const int dk = __builtin_amdgcn_ds_bpermute(4 * (g0 + k), d_j);
#pragma unroll
        for (int e = 0; e < 8; ++e) role[e] = dk >= 0 && dk < D && dk == 8 * j + e ? -2 - k : role[e];
    }
    if (!live) return;
    uint8_t *page = a.pool + id * a.page_bytes;
    const v4 *ksrc = (const v4 *)(a.kp + nh * B * 64);
    v4 *kdst = (v4 *)(page + h * B * 64);
#pragma unroll
    for (int i = j; i < B * 4; i += 16) kdst[i] = ksrc[i];
    const v4 *vsrc = (const v4 *)(a.vp + nh * B * 32);
    v4 *vdst = (v4 *)(page + a.off.vp + h * B * 32);
#pragma unroll
    for (int i = j; i < B * 2; i += 16) vdst[i] = vsrc[i];
    // value scales and offsets: B * 4 bytes each, B / 4 chunks
    if (j < B / 4) {
        ((v4 *)(page + a.off.vs + h * B * 4))[j] = ((const v4 *)(a.vs + nh * B * 2))[j];
        ((v4 *)(page + a.off.vo + h * B * 4))[j] = ((const v4 *)(a.vo + nh * B * 2))[j];
    }
    const v4 *kssrc = (const v4 *)(a.ks + nh * D);
    v4 *ksdst = (v4 *)(page + a.off.ks + h * D * 4);
    ksdst[j] = kssrc[j];
    ksdst[j + 16] = kssrc[j + 16];
    if (j < SPG / 4) ((v4 *)(page + a.off.kp + h * SPG * 4))[j] = ((const v4 *)(a.kpad + nh * SPG))[j];
    uint32_t rw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) rw[q] = (uint32_t)(uint16_t)role[2 * q] | ((uint32_t)(uint16_t)role[2 * q + 1] << 16);
    ((v4 *)(page + a.off.km + h * D * 2))[j] = v4{rw[0], rw[1], rw[2], rw[3]};
}

// ------------------------------------------------------------------ unpack

struct UnpackArgs {
    const uint8_t *pages;              // [n, page_bytes] contiguous
    int64_t H, B, page_bytes;
    PageOffsets off;
    void *k, *v;                       // [n, H, B, 128] of out_dt
    int out_dt;
};

// grid (n * H, B): one workgroup decodes one token of one (page, head).
__global__ __launch_bounds__(128) void unpack_pages_kernel(UnpackArgs a)
{
    const int64_t nh = blockIdx.x, t = blockIdx.y;
    const int64_t n = nh / a.H, h = nh % a.H;
    const int c = threadIdx.x;
    const uint8_t *page = a.pages + n * a.page_bytes;
    const uint8_t *row = page + (h * a.B + t) * 64;
    const int16_t role = ((const int16_t *)(page + a.off.km))[h * D + c];
    const float scale = ((const float *)(page + a.off.ks))[h * D + c];
    const int slot = (row[c >> 1] >> ((c & 1) * 4)) & 15;
    float kv;
    if (role >= 0 && role < D) {
        const int lo = (row[role >> 1] >> ((role & 1) * 4)) & 15;
        kv = __fmul_rn((float)(((slot << 4) | lo) - 128), scale);
    } else if (role <= -2 && role >= -2 - (SPG - 1)) {
        kv = ((const float *)(page + a.off.kp))[h * SPG + (-2 - role)];
    } else {
        kv = __fmul_rn((float)(slot - 8), scale);
    }
    const int64_t o = (nh * a.B + t) * D + c;
    iq_store_as(a.k, o, kv, a.out_dt);
    const uint8_t vb = page[a.off.vp + (h * a.B + t) * 32 + (c >> 2)];
    const int code = (vb >> (2 * (c & 3))) & 3;
    const int64_t pi = (h * a.B + t) * 2 + (c >> 6);
    const float sc = iq_f16_to_f32(((const uint16_t *)(page + a.off.vs))[pi]);
    const float of = iq_f16_to_f32(((const uint16_t *)(page + a.off.vo))[pi]);
    iq_store_as(a.v, o, __fadd_rn(__fmul_rn((float)code, sc), of), a.out_dt);
}

// 16-byte aligned outputs (every supported page size): grid (token tiles
// of UP_TOKENS, pages * H); thread (token, j), j < 16, decodes channels
// 8 j .. 8 j + 7 of one token's key and value.  The page's role map, scales
// and paddings are staged once in LDS.  Keys as k4_decode_rows: each slot is
// one product code * f (a plain channel code = slot - 8, f its scale; a
// source code = 16 slot + lo - 128, lo its donor channel's nibble, from this
// lane's payload word or the word another lane of the token holds; a donor
// code 1, f its padding); values code * scale + offset.  All of a thread's
// page loads are issued first; the outputs go out as non-temporal stores.
constexpr int UP_TOKENS = 128;
constexpr int UP_ITER = UP_TOKENS / 16;            // tokens per thread

template <int OUT>
__device__ __forceinline__ void store8(void *base, int64_t at, const float (&v)[8])
{
    typedef __attribute__((ext_vector_type(4))) uint32_t w4;
    if constexpr (OUT == IQ_F32) {
        w4 *o = (w4 *)((float *)base + at);
        __builtin_nontemporal_store(w4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                       __float_as_uint(v[3])}, o);
        __builtin_nontemporal_store(w4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                                       __float_as_uint(v[7])}, o + 1);
    } else {
        uint32_t h[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) h[k] = pack2<OUT == IQ_F16>(v[2 * k], v[2 * k + 1]);
        __builtin_nontemporal_store(w4{h[0], h[1], h[2], h[3]}, (w4 *)((uint16_t *)base + at));
    }
}

template <int OUT>
__global__ __launch_bounds__(256) void unpack_rows_kernel(UnpackArgs a)
{
    __shared__ float s_scale[D], s_pad[SPG];
    __shared__ int16_t s_role[D];
    const int tid = threadIdx.x, lane = tid & 63, j = tid & 15;
    const int64_t nh = blockIdx.y, n = nh / a.H, h = nh % a.H;
    const uint8_t *page = a.pages + n * a.page_bytes;
    const int B = (int)a.B, t0 = blockIdx.x * UP_TOKENS;
    const int nt = min(UP_TOKENS, B - t0);
    uint32_t kw[UP_ITER], vw[UP_ITER], vp[UP_ITER][2];
#pragma unroll
    for (int i = 0; i < UP_ITER; ++i) {
        const int t = t0 + min((tid >> 4) + 16 * i, nt - 1);      // clamped: every load valid
        const int64_t r = h * B + t;
        kw[i] = *(const uint32_t *)(page + r * 64 + 4 * j);
        vw[i] = *(const uint16_t *)(page + a.off.vp + r * 32 + 2 * j);
        vp[i][0] = ((const uint16_t *)(page + a.off.vs))[r * 2 + (j >> 3)];
        vp[i][1] = ((const uint16_t *)(page + a.off.vo))[r * 2 + (j >> 3)];
    }
    if (tid < D) {
        s_scale[tid] = ((const float *)(page + a.off.ks))[h * D + tid];
        s_role[tid] = ((const int16_t *)(page + a.off.km))[h * D + tid];
    }
    if (tid < SPG) s_pad[tid] = ((const float *)(page + a.off.kp))[h * SPG + tid];
    __syncthreads();
    uint32_t m[8], lo_at[8], lo_w[8];
    int off[8], bp[8];
    bool xl[8];
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int rl = s_role[8 * j + e];
        const bool src = rl >= 0 && rl < D, don = rl <= -2 && rl >= -2 - (SPG - 1);
        f[e] = don ? s_pad[-2 - rl] : s_scale[8 * j + e];
        m[e] = src ? 16u : don ? 0u : 1u;
        off[e] = src ? 128 : don ? -1 : 8;
        lo_w[e] = src ? 4u : 0u;
        lo_at[e] = src ? 4u * (uint32_t)(rl & 7) : 0u;
        xl[e] = src && (rl >> 3) != j;
        bp[e] = 4 * ((lane & ~15) | (src ? rl >> 3 : 0));
    }
#pragma unroll
    for (int i = 0; i < UP_ITER; ++i) {
        const int tt = (tid >> 4) + 16 * i;
        const uint32_t w = kw[i];
        uint32_t x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (uint32_t)__builtin_amdgcn_ds_bpermute(bp[e], (int)w);
        if (tt >= nt) continue;
        const int64_t o = (nh * B + t0 + tt) * D + 8 * j;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t wd = xl[e] ? x[e] : w;
            const uint32_t slot = __builtin_amdgcn_ubfe(w, 4 * e, 4);
            const uint32_t lo = __builtin_amdgcn_ubfe(wd, lo_at[e], lo_w[e]);
            v[e] = __fmul_rn((float)((int)(__umul24(slot, m[e]) + lo) - off[e]), f[e]);
        }
        store8<OUT>(a.k, o, v);
        const float sc = iq_f16_to_f32((uint16_t)vp[i][0]), of = iq_f16_to_f32((uint16_t)vp[i][1]);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            v[e] = __fadd_rn(__fmul_rn((float)((vw[i] >> (2 * e)) & 3u), sc), of);
        store8<OUT>(a.v, o, v);
    }
}

// Pages of B = 16, 32 or 64 tokens: each 16-lane group takes one (page,
// head) and all its tokens, 16 at a time (loads first), lane j channels
// 8 j .. 8 j + 7.  Lane j reads its own eight roles and scales and padding j
// of the page straight from the page (no LDS, no barrier); a donor slot
// takes its padding from the lane of its group that read it.  Same
// arithmetic as unpack_rows_kernel.
template <int OUT, int B>
__global__ __launch_bounds__(256) void unpack_small_pages_kernel(UnpackArgs a, int64_t nph)
{
    typedef __attribute__((ext_vector_type(4))) uint32_t w4;
    const int tid = threadIdx.x, lane = tid & 63, j = tid & 15;
    const int64_t ph = (int64_t)blockIdx.x * 16 + (tid >> 4);
    const bool ok = ph < nph;                                    // group-uniform
    const int64_t phc = ok ? ph : nph - 1;
    const int64_t n = phc / a.H, h = phc % a.H;
    const uint8_t *page = a.pages + n * a.page_bytes;
    const w4 rw = *(const w4 *)(page + a.off.km + (h * D + 8 * j) * 2);          // roles 8 j .. 8 j + 7
    const w4 s0 = *(const w4 *)(page + a.off.ks + (h * D + 8 * j) * 4);
    const w4 s1 = *(const w4 *)(page + a.off.ks + (h * D + 8 * j + 4) * 4);
    const float pad_j = ((const float *)(page + a.off.kp))[h * SPG + j];
    uint32_t m[8], lo_at[8], lo_w[8];
    int off[8], bp[8];
    bool xl[8];
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int rl = (int)(int16_t)(rw[e >> 1] >> (16 * (e & 1)));
        const bool src = rl >= 0 && rl < D, don = rl <= -2 && rl >= -2 - (SPG - 1);
        const float pad = __int_as_float(
            __builtin_amdgcn_ds_bpermute(4 * ((lane & ~15) | (don ? -2 - rl : 0)), __float_as_int(pad_j)));
        f[e] = don ? pad : __uint_as_float(e < 4 ? s0[e] : s1[e - 4]);
        m[e] = src ? 16u : don ? 0u : 1u;
        off[e] = src ? 128 : don ? -1 : 8;
        lo_w[e] = src ? 4u : 0u;
        lo_at[e] = src ? 4u * (uint32_t)(rl & 7) : 0u;
        xl[e] = src && (rl >> 3) != j;
        bp[e] = 4 * ((lane & ~15) | (src ? rl >> 3 : 0));
    }
#pragma unroll 1
    for (int c = 0; c < B; c += 16) {
        uint32_t kw[16], vw[16], vp[16][2];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int64_t r = h * B + c + i;
            kw[i] = *(const uint32_t *)(page + r * 64 + 4 * j);
            vw[i] = *(const uint16_t *)(page + a.off.vp + r * 32 + 2 * j);
            vp[i][0] = ((const uint16_t *)(page + a.off.vs))[r * 2 + (j >> 3)];
            vp[i][1] = ((const uint16_t *)(page + a.off.vo))[r * 2 + (j >> 3)];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t w = kw[i];
            uint32_t x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = (uint32_t)__builtin_amdgcn_ds_bpermute(bp[e], (int)w);
            if (!ok) continue;
            const int64_t o = (phc * B + c + i) * D + 8 * j;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t wd = xl[e] ? x[e] : w;
                const uint32_t slot = __builtin_amdgcn_ubfe(w, 4 * e, 4);
                const uint32_t lo = __builtin_amdgcn_ubfe(wd, lo_at[e], lo_w[e]);
                v[e] = __fmul_rn((float)((int)(__umul24(slot, m[e]) + lo) - off[e]), f[e]);
            }
            store8<OUT>(a.k, o, v);
            const float sc = iq_f16_to_f32((uint16_t)vp[i][0]), of = iq_f16_to_f32((uint16_t)vp[i][1]);
#pragma unroll
            for (int e = 0; e < 8; ++e)
                v[e] = __fadd_rn(__fmul_rn((float)((vw[i] >> (2 * e)) & 3u), sc), of);
            store8<OUT>(a.v, o, v);
        }
    }
}

template <int OUT>
void launch_unpack(const UnpackArgs &a, int64_t nph, hipStream_t st)
{
    const dim3 small((unsigned)((nph + 15) / 16));
    switch (a.B) {
    case 16: hipLaunchKernelGGL((unpack_small_pages_kernel<OUT, 16>), small, dim3(256), 0, st, a, nph); break;
    case 32: hipLaunchKernelGGL((unpack_small_pages_kernel<OUT, 32>), small, dim3(256), 0, st, a, nph); break;
    case 64: hipLaunchKernelGGL((unpack_small_pages_kernel<OUT, 64>), small, dim3(256), 0, st, a, nph); break;
    default:
        hipLaunchKernelGGL((unpack_rows_kernel<OUT>), dim3((unsigned)((a.B + UP_TOKENS - 1) / UP_TOKENS), (unsigned)nph),
                           dim3(256), 0, st, a);
    }
}

// ------------------------------------------------------------------ decode

struct PagedArgs {
    const uint16_t *q;                 // [seq, Hq, 128] bf16 (element strides below)
    int64_t q_ss, q_sh;
    int G, H, B;
    const uint8_t *pool;
    int64_t page_bytes, pool_pages;
    PageOffsets off;
    const int32_t *bt;                 // block tables [seq, bt_ss]
    int64_t bt_ss, max_pages;
    const int32_t *seq_info;           // [seq, 3] (pages, tail, sink) or null
    int npg0, tail0, sink0;            // used when seq_info is null
    const uint16_t *dense;             // [slots, 2, H, B + 4, 128] bf16
    int64_t dense_ss;
    const int32_t *dense_slots;        // dense slot of each sequence, or null (slot = sequence)
    // optional compacted work list: grid row y is (sequence work[y] >> 16,
    // partition work[y] & 0xffff), only live partitions; null: row y is
    // partition y of sequence blockIdx.z
    const int32_t *work;
    int n_seq;
    int max_parts;
    float c_log2;                      // softmax scale * log2(e)
    float *ws;                         // seq * Hq * max_parts partials (Partials layout)
};

struct SeqGeom {
    int npg, tail, sink, npp, ndp;
};

__device__ __forceinline__ SeqGeom seq_geom(const PagedArgs &a, int s)
{
    SeqGeom g;
    if (a.seq_info) {
        g.npg = a.seq_info[3 * s];
        g.tail = a.seq_info[3 * s + 1];
        g.sink = a.seq_info[3 * s + 2];
    } else {
        g.npg = a.npg0;
        g.tail = a.tail0;
        g.sink = a.sink0;
    }
    g.npg = max(0, min(g.npg, (int)a.max_pages));
    g.tail = max(0, min(g.tail, a.B));
    g.sink = max(0, min(g.sink, 4));
    g.npp = (g.npg * a.B + PART - 1) / PART;
    g.ndp = (a.B + 4 + PART - 1) / PART;
    return g;
}

// Pages a wavefront's 64 tokens touch, and the first of them.
__host__ __device__ constexpr int pages_per_wave(int npg) { return npg >= WAVES ? npg / WAVES : 1; }
__device__ __forceinline__ int page_of_wave(int npg, int wave)
{
    return npg >= WAVES ? wave * (npg / WAVES) : wave * npg / WAVES;
}

// Workgroup LDS of decode_paged, shared by its packed and dense bodies.
// Each wavefront's slot of v (SLOT bytes) holds in turn: the K constant
// pairs of its pages [0, KAP_BYTES) up to Q.K; then the salient selection
// matrix of one page at a time; then its decoded V tiles and its combine
// rows (the whole slot).  At 16-token pages a workgroup takes 40,704 bytes:
// four per compute unit.
constexpr int SLOT = 16 * VR * 4;          // bytes per wavefront slot
constexpr int KAP_GROUP = 34;              // pairs per 32-channel group (+2: the four groups on distinct banks)
constexpr int KAP_PAGE = 4 * KAP_GROUP;    // pairs per page
constexpr int KAP_BYTES = 4 * KAP_PAGE * 8;   // the constant pairs of up to four pages
static_assert(KAP_BYTES <= SLOT, "the constant pairs fit in a wavefront's slot");
static_assert(16 * SELROW <= SLOT, "a page's selection matrix fits in a wavefront's slot");

template <int NPG>
struct __attribute__((aligned(16))) PagedSmem {
    uint32_t v[WAVES][16 * VR];        // per-wavefront slots (above)
    uint16_t q[16 * QROW];
    uint32_t salw[NPG][SPG];           // salient row r of a page: source and donor bytes
    float ssc[NPG][SPG];               // salient row r of a page: the source's scale
    int nsrc[WAVES];                   // sources among a wavefront's channels (pages shared by two wavefronts)
    float wm[WAVES][16], wl[WAVES][16];

    __device__ f32x2 *kap(int w) { return (f32x2 *)&v[w][0]; }                          // [page of w][4][KAP_GROUP]
};

// One partition of one sequence.  The packed and the dense body are separate
// instantiations so that neither has a branch between its loads and their
// first use (a branch join there makes the compiler wait for every load in
// flight).  `pid` holds the block-table entries of this wavefront's pages
// (page_of_wave), read with scalar loads before the sequence lengths were
// known.
template <int NPG, bool PACKED>
__device__ __forceinline__ void paged_body(const PagedArgs &a, PagedSmem<NPG> &sm, const SeqGeom &geo, int wave,
                                           const int (&pid)[pages_per_wave(NPG)], int p, int sq)
{
    constexpr int B = PART / NPG;
    constexpr int VQW = 2;                       // dwords per 32-channel quarter of a V2 row
    constexpr int CPT = (NPG * D + 255) / 256;   // (page, channel) constants per thread
    constexpr int PPW = pages_per_wave(NPG);

    const int tid = threadIdx.x, lane = tid & 63;
    const int gl = lane & 15, ql = lane >> 4;
    const int pl = lane & 15, qq = lane >> 4;      // V writer: pair row pl, channels 32 qq .. 32 qq + 31
    const int h = blockIdx.x;
    const int G = a.G;
    const float unit = fp8x2<false>(1u).x;       // fp8 byte 1 == 2^-9
    const float inv_unit = 1.0f / unit;
    uint32_t *const s_v = &sm.v[0][0];
    uint16_t *const s_q = sm.q;
    const int base = 64 * wave;

    // ---------------- geometry
    int ntok, tok0 = 0, slot0 = 0;
    const uint16_t *dk = nullptr, *dv = nullptr;
    if constexpr (PACKED) {
        tok0 = p * PART;
        ntok = min(PART, geo.npg * B - tok0);
    } else {
        slot0 = (p - geo.npp) * PART;
        ntok = min(PART, B + 4 - slot0);
        const uint16_t *dn = a.dense + (int64_t)(a.dense_slots ? a.dense_slots[sq] : sq) * a.dense_ss;
        dk = dn + ((int64_t)h * (B + 4) + slot0) * D;
        dv = dn + ((int64_t)(a.H + h) * (B + 4) + slot0) * D;
    }
    const int qg = tid >> 4, qc = (tid & 15) * 8;
    const u32x4 qraw = ld16(a.q + sq * a.q_ss + (int64_t)(h * G + (qg < G ? qg : G - 1)) * a.q_sh + qc);

    // ---------------- this wavefront's page addresses, in scalar registers:
    // wpg[i] is page page_of_wave(wave) + i of the partition.  Pages past the
    // partition's end or outside the pool read page 0 and stay dead (bit i of
    // okmask clear).
    const uint8_t *wpg[PPW];
    uint32_t okmask = 0;
    if constexpr (PACKED) {
        const int npg_here = (ntok + B - 1) / B;
#pragma unroll
        for (int i = 0; i < PPW; ++i) {
            const bool ok = page_of_wave(NPG, wave) + i < npg_here && pid[i] >= 0 && pid[i] < a.pool_pages;
            // page_bytes < 2^32 (checked at launch): one 32 x 32 -> 64-bit product
            wpg[i] = a.pool + (uint64_t)(uint32_t)(ok ? pid[i] : 0) * (uint32_t)a.page_bytes;
            okmask |= (ok ? 1u : 0u) << i;
        }
    }
    // (page, channel) of this thread's k-th per-channel constant: each
    // wavefront takes its own pages (NPG >= 4), or half a page (NPG = 2), or
    // waves 0-1 the one page (NPG = 1)
    auto cpage = [&](int k) -> int { return NPG >= WAVES ? k >> 1 : 0; };            // index into wpg
    auto cpart = [&](int k) -> int { return NPG >= WAVES ? wave * PPW + (k >> 1) : (NPG == 2 ? wave >> 1 : 0); };
    auto cchan = [&](int k) -> int { return NPG >= WAVES ? ((k & 1) << 6) + lane : (tid & (D - 1)); };
    const bool cvalid = NPG > 1 || tid < D;

    // ---------------- every global load of the partition, unconditional (clamped)
    float ksc[CPT], kpad = 0.0f;
    int krl[CPT];
    u32x4 kw[4];
    uint32_t vw[2][2][VQW];
    uint32_t vp[2][2][2];                          // f16 bits of the V scale / offset
    if constexpr (PACKED) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            // the page is wave-uniform: scalar base, 32-bit lane offset
            const uint8_t *page = wpg[cpage(k)];
            const int c = cchan(k);
            ksc[k] = ldg_at<float>(page, (uint32_t)(a.off.ks + (h * D + c) * 4));
            krl[k] = ldg_at<int16_t>(page, (uint32_t)(a.off.km + (h * D + c) * 2));
        }
        {
            // lane l of a wavefront: padding j = l % 16 of its page l / 16
            const int lpl = NPG >= WAVES ? min(lane >> 4, PPW - 1) : 0;
            const uint8_t *page = wpg[0];
#pragma unroll
            for (int i = 1; i < PPW; ++i) page = lpl == i ? wpg[i] : page;
            kpad = ldg_at<float>(page, (uint32_t)(a.off.kp + (h * SPG + (lane & 15)) * 4));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // a 16-token tile lies in one page (B is a multiple of 16); rows
            // past the end read a clamped row of that page and stay dead
            const uint8_t *page = wpg[NPG >= WAVES ? (16 * j) / B : 0];
            const uint32_t t = (uint32_t)min(base + 16 * j + gl, ntok - 1) & (B - 1);
            kw[j] = ldnt_at<u32x4>(page, (uint32_t)((h * B + t) * 64 + 16 * ql));
        }
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                // pair row pl of half m: tokens 32 m + pl (u = 0) and + 16 (u = 1),
                // each run of 16 tokens inside one page
                const uint8_t *page = wpg[NPG >= WAVES ? (32 * m + 16 * u) / B : 0];
                const uint32_t r = (uint32_t)(h * B) + ((uint32_t)min(base + 32 * m + 16 * u + pl, ntok - 1) & (B - 1));
                const u32x2 w = ldnt_at<u32x2>(page, (uint32_t)a.off.vp + r * 32 + 8 * qq);
                vw[m][u][0] = w[0];
                vw[m][u][1] = w[1];
                vp[m][u][0] = ldg_at<uint16_t>(page, (uint32_t)a.off.vs + (r * 2 + (qq >> 1)) * 2);
                vp[m][u][1] = ldg_at<uint16_t>(page, (uint32_t)a.off.vo + (r * 2 + (qq >> 1)) * 2);
            }
        // keep every use of the constants below the payload issue
        asm volatile("" ::: "memory");
    }

    // ---------------- query rows; per-page constants and roles
    // Wavefront w reads the K constants of page lp from its slot: wavefronts
    // own their pages (NPG >= 4), or share the one page of their tokens.
    auto owner0 = [&](int lp) -> int { return NPG >= WAVES ? lp / PPW : lp * WAVES / NPG; };
    constexpr int OWNERS = NPG >= WAVES ? 1 : WAVES / NPG;
    auto local = [&](int lp) -> int { return NPG >= WAVES ? lp % PPW : 0; };
    *(u32x4 *)(s_q + qg * QROW + qc) = qg < G ? qraw : u32x4{0u, 0u, 0u, 0u};
    if constexpr (PACKED) {
        // Roles come from the page's role map, as the reference decodes a
        // page (role >= 0: a source, whose donor is channel `role`; role
        // <= -2: donor -2 - role; -1: a normal channel), with no descriptor
        // lists:
        // * a normal channel gets the pair (s * 2^9, -8 s);
        // * a source gets (0, 0) and takes the salient row of its rank among
        //   the page's sources in channel order (ballots), where it records
        //   its own and its donor's byte for the selection matrix and its
        //   scale; rows past the page's source count keep bytes 0, scale 0;
        // * donor j gets (0, pad_j), pad_j read from the lane that loaded it,
        //   so Q.K itself adds q . round(pad_j).
        // Pages of at most 64 tokens belong to one wavefront each, which
        // resolves them alone; a longer page is shared by two wavefronts
        // (channels 0-63 and 64-127), the second adding the first's source
        // count to its ranks.
        uint64_t msk[CPT];
#pragma unroll
        for (int k = 0; k < CPT; ++k) msk[k] = __ballot(cvalid && krl[k] >= 0 && krl[k] < D);
        if constexpr (NPG >= WAVES) {
            if (lane < 16 * PPW) {
                sm.salw[wave * PPW + (lane >> 4)][lane & 15] = 0u;
                sm.ssc[wave * PPW + (lane >> 4)][lane & 15] = 0.0f;
            }
            wave_lds_sync();
        } else {
            if (tid < NPG * SPG) {
                sm.salw[tid / SPG][tid % SPG] = 0u;
                sm.ssc[tid / SPG][tid % SPG] = 0.0f;
            }
            if (lane == 0) sm.nsrc[wave] = (int)__popcll(msk[0]);
            __syncthreads();
        }
        if (cvalid) {
#pragma unroll
            for (int k = 0; k < CPT; ++k) {
                const int lp = cpart(k), c = cchan(k), role = krl[k], j = -2 - role;
                int rank = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(msk[k] >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((uint32_t)msk[k], 0u));
                if constexpr (NPG >= WAVES) {
                    if (k & 1) rank += (int)__popcll(msk[k - 1]);
                } else if (wave & 1) {
                    rank += sm.nsrc[wave - 1];
                }
                const bool donor = j >= 0 && j < SPG;
                const int pad_lane = (NPG >= WAVES ? 16 * cpage(k) : 0) + (donor ? j : 0);
                const float pad = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * pad_lane, __float_as_int(kpad)));
                const float A = role == -1 ? ksc[k] * inv_unit : 0.0f;
                const f32x2 pair = {A, role == -1 ? A * -0.015625f : (donor ? pad : 0.0f)};   // (s * 2^9, -8 s) exact
#pragma unroll
                for (int o = 0; o < OWNERS; ++o)
                    sm.kap(owner0(lp) + o)[local(lp) * KAP_PAGE + (c >> 5) * KAP_GROUP + (c & 31)] = pair;
                if (role >= 0 && role < D && rank < SPG) {
                    sm.salw[lp][rank] = (uint32_t)(c >> 1) | ((uint32_t)((c & 1) * 4) << 8) |
                                        ((uint32_t)(role >> 1) << 16) | ((uint32_t)((role & 1) * 4) << 24);
                    sm.ssc[lp][rank] = ksc[k];
                }
            }
        }
    }
    __syncthreads();

    u32x4 qb[4];                                   // B operand: Q[g = gl][32 ql + 8 d + e]
#pragma unroll
    for (int d = 0; d < 4; ++d) qb[d] = *(const u32x4 *)(s_q + gl * QROW + 32 * ql + 8 * d);

    float m_run = NEG_INF, l_run = 0.0f;
    f32x4 acc[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t *vt = s_v + wave * (16 * VR);
    // The P.V operand reads: volatile, so that each lane's four pair rows
    // stay four single-dword LDS reads straight into the operand registers
    // (the compiler would otherwise pair the reads of channel tiles n and
    // n + 1 and copy every operand into place).
    const volatile __attribute__((address_space(3))) uint32_t *const vtile =
        (const volatile __attribute__((address_space(3))) uint32_t *)vt;

    if (base < ntok) {
        // a token is live when it exists in this partition and (packed) lies
        // in a live page past the sink, or (dense) is a sink slot or a tail
        // slot whose position is past the sink (kernels.py:37,48)
        auto live = [&](int t) -> bool {
            if (t >= ntok) return false;
            if constexpr (PACKED) return ((okmask >> ((uint32_t)(t - base) / B)) & 1u) && tok0 + t >= geo.sink;
            const int slot = slot0 + t;
            return slot < geo.sink || (slot >= 4 && slot < 4 + geo.tail && geo.npg * B + slot - 4 >= geo.sink);
        };
        f32x4 sc[4];
        if constexpr (PACKED) {
            const f32x2 *kap = sm.kap(wave);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int lpl = NPG >= WAVES ? (16 * j) / B : 0;   // the tile's page among the wavefront's
                asm volatile("" ::: "memory");
                f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const f32x2 *cp = kap + lpl * KAP_PAGE + ql * KAP_GROUP + 8 * d;
                    float A[8], Bc[8];
#pragma unroll
                    for (int e2 = 0; e2 < 4; ++e2) {
                        const u32x4 c = *(const u32x4 *)(cp + 2 * e2);   // pairs 2 e2, 2 e2 + 1
                        A[2 * e2] = __uint_as_float(c[0]);
                        Bc[2 * e2] = __uint_as_float(c[1]);
                        A[2 * e2 + 1] = __uint_as_float(c[2]);
                        Bc[2 * e2 + 1] = __uint_as_float(c[3]);
                    }
                    const uint32_t x = kw[j][d];
                    const uint32_t lo = x & 0x0f0f0f0fu, hi = (x >> 4) & 0x0f0f0f0fu;
                    const f32x2 e01 = fp8x2<false>(lo), e23 = fp8x2<true>(lo);
                    const f32x2 o01 = fp8x2<false>(hi), o23 = fp8x2<true>(hi);
                    u32x4 kv;
                    kv[0] = pack2<false>(fmaf(e01.x, A[0], Bc[0]), fmaf(o01.x, A[1], Bc[1]));
                    kv[1] = pack2<false>(fmaf(e01.y, A[2], Bc[2]), fmaf(o01.y, A[3], Bc[3]));
                    kv[2] = pack2<false>(fmaf(e23.x, A[4], Bc[4]), fmaf(o23.x, A[5], Bc[5]));
                    kv[3] = pack2<false>(fmaf(e23.y, A[6], Bc[6]), fmaf(o23.y, A[7], Bc[7]));
                    s = mma32<false>(kv, qb[d], s);
                }
                sc[j] = s;
            }
            // salient terms: the codes 16 hi + lo - 128 come from two int8
            // products of the page's selection matrix (row k: 16 at the byte of
            // descriptor k's source, 1 at its donor's; channel c at byte
            // (c & 1) * 64 + c / 2) with the tile's nibble planes, so lane
            // (token gl, ql) receives the codes of descriptors 4 ql + r: the A
            // operand of the salient product.  The matrix is built in this
            // wavefront's slot (free after Q.K), one page at a time: each new
            // page clears the previous page's 32 bytes and sets its own.
            uint8_t *const ssel = (uint8_t *)vt;
#pragma unroll
            for (int i = lane; i < 16 * SELROW / 16; i += 64) *(u32x4 *)(ssel + 16 * i) = u32x4{0u, 0u, 0u, 0u};
            wave_lds_sync();
            uint32_t mark = 0;                          // lanes 0-31: the byte this lane set
            i32x4 sel_lo = {0, 0, 0, 0}, sel_hi = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int lp = (base + 16 * j) / B;
                if (j == 0 || (16 * j) % B == 0) {      // the tile starts a page
                    if (lane < 32) {
                        const uint32_t w = sm.salw[lp][lane & 15];
                        const uint32_t f = lane < 16 ? w & 0xffffu : w >> 16;      // (byte, 4 * parity)
                        const uint32_t at = (lane & 15) * SELROW + (f & 0xffu) + ((f >> 8) << 4);
                        if (j > 0) ssel[mark] = 0;
                        ssel[at] = lane < 16 ? 16 : 1;
                        mark = at;
                    }
                    wave_lds_sync();
                    sel_lo = *(const i32x4 *)(ssel + gl * SELROW + 16 * ql);
                    sel_hi = *(const i32x4 *)(ssel + gl * SELROW + D / 2 + 16 * ql);
                }
                i32x4 lo4, hi4;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    lo4[d] = (int)(kw[j][d] & 0x0f0f0f0fu);
                    hi4[d] = (int)((kw[j][d] >> 4) & 0x0f0f0f0fu);
                }
                i32x4 code = __builtin_amdgcn_mfma_i32_16x16x64_i8(sel_lo, lo4, i32x4{-128, -128, -128, -128}, 0, 0, 0);
                code = __builtin_amdgcn_mfma_i32_16x16x64_i8(sel_hi, hi4, code, 0, 0, 0);
                const f32x4 ssc = *(const f32x4 *)&sm.ssc[lp][4 * ql];
                float v[4];
                uint32_t qv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // Q[g][source channel]; the source is 2 (w & 255) + ((w >> 8) & 255) / 4
                    const uint32_t w = sm.salw[lp][4 * ql + e];
                    qv[e] = s_q[gl * QROW + 2 * (w & 0xffu) + (((w >> 8) & 0xffu) >> 2)];
                    // (code - 128) * s in one rounding, as the reference's multiply
                    v[e] = (float)code[e] * ssc[e];
                }
                const u32x2 ka = {pack2<false>(v[0], v[1]), pack2<false>(v[2], v[3])};
                const u32x2 qs = {qv[0] | (qv[1] << 16), qv[2] | (qv[3] << 16)};
                sc[j] = mma16<false>(ka, qs, sc[j]);
            }
        } else {
            // dense sink / tail slots: bf16 rows are the A operand directly;
            // rows of dead slots are zeroed (the buffer may hold NaN there)
#pragma unroll
            for (int j2 = 0; j2 < 4; j2 += 2) {
                u32x4 kd[2][4];
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const int t = min(base + 16 * (j2 + jj) + gl, ntok - 1);
#pragma unroll
                    for (int d = 0; d < 4; ++d) kd[jj][d] = ld16(dk + (int64_t)t * D + 32 * ql + 8 * d);
                }
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const bool ok = live(base + 16 * (j2 + jj) + gl);
                    f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int d = 0; d < 4; ++d) s = mma32<false>(ok ? kd[jj][d] : u32x4{0u, 0u, 0u, 0u}, qb[d], s);
                    sc[j2 + jj] = s;
                }
            }
        }

        // ---------------- softmax (log2 domain); lane holds g = gl, tokens 16 j + 4 ql + r.
        // Raw logits: the scale is positive, so the maximum commutes with it
        // and p = 2^(s c - m) takes one fma per logit.
        // (wave-uniform) every token of this wavefront is live: no masking
        const bool all_live = PACKED && okmask == (1u << PPW) - 1u && base + 64 <= ntok && tok0 + base >= geo.sink;
        if (!all_live) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (!live(base + 16 * j + 4 * ql + r)) sc[j][r] = NEG_INF;
        }
        float cmax = NEG_INF;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) cmax = fmaxf(cmax, sc[j][r]);
        const float m_new = xmax16(cmax) * a.c_log2;
        const float m_use = m_new == NEG_INF ? 0.0f : m_new;
        float lsum = 0.0f;
        float pr[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pr[j][r] = __builtin_amdgcn_exp2f(fmaf(sc[j][r], a.c_log2, -m_use));
                lsum += pr[j][r];
            }
        // B operand of half chunk m: k-slot pair r = tokens 32 m + 4 ql + r and
        // 32 m + 16 + 4 ql + r (tiles 2 m and 2 m + 1)
        u32x4 phi[2], plo[2];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t hh = pack2<false>(pr[2 * m][r], pr[2 * m + 1][r]);
                phi[m][r] = hh;
                plo[m][r] = pack2<false>(pr[2 * m][r] - to_f32<false>(hh & 0xffffu),
                                         pr[2 * m + 1][r] - to_f32<false>(hh >> 16));
            }
        l_run = lsum;
        m_run = m_new;

        // ---------------- two half chunks: decode 32 V rows to LDS, then O^T += V^T P^T
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            uint32_t *dst = vt + pl * VR + 32 * qq;    // pair row pl, channels 32 qq .. 32 qq + 31
            if (m > 0) wave_lds_sync();                // every lane has read half chunk m - 1
            if constexpr (PACKED) {
                // dead tokens decode to zero: a zero weight times a non-finite
                // value (a page outside the pool) would still poison P.V
                float s9[2], of[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const bool ok = live(base + 32 * m + 16 * u + pl);
                    s9[u] = ok ? iq_f16_to_f32((uint16_t)vp[m][u][0]) * inv_unit : 0.0f;
                    of[u] = ok ? iq_f16_to_f32((uint16_t)vp[m][u][1]) : 0.0f;
                }
#pragma unroll
                for (int w = 0; w < 2; ++w) {          // 16 channels 32 qq + 16 w + (4 b + k)
                    float val[2][16];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const uint32_t x = vw[m][u][w];
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const uint32_t b = (x >> (2 * k)) & 0x03030303u;
                            const f32x2 c0 = fp8x2<false>(b), c1 = fp8x2<true>(b);
                            val[u][k] = fmaf(c0.x, s9[u], of[u]);
                            val[u][4 + k] = fmaf(c0.y, s9[u], of[u]);
                            val[u][8 + k] = fmaf(c1.x, s9[u], of[u]);
                            val[u][12 + k] = fmaf(c1.y, s9[u], of[u]);
                        }
                    }
#pragma unroll
                    for (int c4 = 0; c4 < 4; ++c4) {
                        u32x4 o;
#pragma unroll
                        for (int i = 0; i < 4; ++i) o[i] = pack2<false>(val[0][4 * c4 + i], val[1][4 * c4 + i]);
                        *(u32x4 *)(dst + 16 * w + 4 * c4) = o;
                    }
                }
            } else {
                const int t0 = base + 32 * m + pl, t1 = t0 + 16;
                const int ta = min(t0, ntok - 1), tb = min(t1, ntok - 1);
                const bool oka = live(t0), okb = live(t1);
                u32x4 r0[4], r1[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    r0[i] = ld16(dv + (int64_t)ta * D + 32 * qq + 8 * i);
                    r1[i] = ld16(dv + (int64_t)tb * D + 32 * qq + 8 * i);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (!oka) r0[i] = u32x4{0u, 0u, 0u, 0u};
                    if (!okb) r1[i] = u32x4{0u, 0u, 0u, 0u};
                    u32x4 lo, hi;
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        lo[w] = __builtin_amdgcn_perm(r1[i][w], r0[i][w], 0x05040100u);   // (r0.lo, r1.lo)
                        hi[w] = __builtin_amdgcn_perm(r1[i][w], r0[i][w], 0x07060302u);   // (r0.hi, r1.hi)
                    }
                    *(u32x4 *)(dst + 8 * i) = u32x4{lo[0], hi[0], lo[1], hi[1]};
                    *(u32x4 *)(dst + 8 * i + 4) = u32x4{lo[2], hi[2], lo[3], hi[3]};
                }
            }
            wave_lds_sync();                           // the tile's rows come from other lanes
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                u32x4 va;                              // k-slot pair r: pair row 4 ql + r
#pragma unroll
                for (int r = 0; r < 4; ++r) va[r] = vtile[(4 * ql + r) * VR + 16 * n + gl];
                acc[n] = mma32<false>(va, phi[m], acc[n]);
                acc[n] = mma32<false>(va, plo[m], acc[n]);
            }
        }
    }

    // ---------------- combine the four wavefronts, write this partition's partial
    // Each wavefront stages its unnormalized O as O[g][c] rows next to its
    // (m, l); a reader weights the four rows by 2^(m_w - max m) and adds.
    l_run = xsum16(l_run);
    if (ql == 0) {
        sm.wm[wave][gl] = m_run;
        sm.wl[wave][gl] = l_run;
    }
    float *ot = (float *)vt;
#pragma unroll
    for (int n = 0; n < 8; ++n) *(f32x4 *)(ot + gl * OROW + 16 * n + 4 * ql) = acc[n];
    __syncthreads();
    for (int i = tid; i < G * (D / 4); i += 256) {
        const int g = i >> 5, c = (i & 31) * 4;
        float mw[WAVES], mx = NEG_INF;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            mw[w] = sm.wm[w][g];
            mx = fmaxf(mx, mw[w]);
        }
        f32x4 num = {0.0f, 0.0f, 0.0f, 0.0f};
        float den = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float wt = mw[w] == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - mx);
            const f32x4 o = *(const f32x4 *)((const float *)sm.v[w] + g * OROW + c);
#pragma unroll
            for (int e = 0; e < 4; ++e) num[e] = fmaf(o[e], wt, num[e]);
            den = fmaf(sm.wl[w][g], wt, den);
        }
        const Partials pt = partials(a.ws, (int64_t)a.n_seq * a.H * G * a.max_parts);
        const int64_t row = ((int64_t)sq * a.H * G + h * G + g) * a.max_parts + p;
        *(f32x4 *)(pt.o + row * D + c) = num;
        if (c == 0) pt.ml[row] = f32x2{mx == NEG_INF ? NEG_INF : mx * LN2, den};
    }
}

// One workgroup per (KV head, partition, sequence); NPG = pages per packed
// partition (PART / B).
template <int NPG>
__global__ __launch_bounds__(256, 4) void decode_paged(PagedArgs a)
{
    constexpr int PPW = pages_per_wave(NPG);
    __shared__ PagedSmem<NPG> sm;
    int p = blockIdx.y, sq = blockIdx.z;
    if (a.work) {
        const int item = a.work[blockIdx.y];
        sq = item >> 16;
        p = item & 0xffff;
        if (sq >= a.n_seq || p >= a.max_parts) return;     // an item outside the batch does nothing
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // this wavefront's block-table entries (scalar loads), requested before
    // the lengths arrive; the last partition of a table clamps its indices
    int pid[PPW];
    const int64_t first = (int64_t)p * NPG + page_of_wave(NPG, wave);
    const int32_t *row = a.bt + sq * a.bt_ss;
    if (first + PPW <= a.max_pages) {
#pragma unroll
        for (int i = 0; i < PPW; ++i) pid[i] = row[first + i];
    } else {
#pragma unroll
        for (int i = 0; i < PPW; ++i) pid[i] = a.max_pages > 0 ? row[min(first + i, a.max_pages - 1)] : -1;
    }
    const SeqGeom geo = seq_geom(a, sq);
    if (p >= geo.npp + geo.ndp) return;
    if (p < geo.npp) paged_body<NPG, true>(a, sm, geo, wave, pid, p, sq);
    else paged_body<NPG, false>(a, sm, geo, wave, pid, p, sq);
}

// grid (64 * ceil(Hq / 8), 1, seq) of single-wave workgroups: merges the
// partitions of one sequence for 16 channels of one query head (the eight
// channel slices of a head on one XCD), as decode_reduce: lane (column c4 of
// four channels, partition lane part) takes every 16th partition from
// `part`, a 16-byte load of its channels and an 8-byte load of (m, l) each,
// nine partitions per round all in flight; the 16 states of a column then
// merge inside the wave (DPP row rotations and permlane swaps), with no LDS
// and no barrier (four-wave workgroups of four slices each measured no
// faster).
__global__ __launch_bounds__(64) void paged_reduce(PagedArgs a, void *out, int64_t out_ss, int odt)
{
    constexpr int BATCH = 9;
    int hq, slice;
    iq_xcd_item_slice((int)blockIdx.x, hq, slice);       // the 8 channel slices of a head on one XCD
    if (hq >= a.H * a.G) return;
    const int sq = blockIdx.z;
    const int lane = threadIdx.x, c4 = lane & 3, part = lane >> 2;
    const int c0 = slice * 16 + 4 * c4;
    const SeqGeom geo = seq_geom(a, sq);
    const int P = geo.npp + geo.ndp;
    const Partials pt = partials(a.ws, (int64_t)a.n_seq * a.H * a.G * a.max_parts);
    const int64_t row0 = ((int64_t)sq * a.H * a.G + hq) * a.max_parts;
    float m = NEG_INF, den = 0.0f;
    f32x4 num = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int p0 = part; p0 < P; p0 += 16 * BATCH) {
        // every load of the round first, the masks after (see decode_reduce)
        f32x4 ov[BATCH];
        f32x2 ml[BATCH];
#pragma unroll
        for (int k = 0; k < BATCH; ++k) {
            const int64_t row = row0 + min(p0 + 16 * k, P - 1);
            ov[k] = *(const f32x4 *)(pt.o + row * D + c0);
            ml[k] = pt.ml[row];
        }
        float mm = m;
#pragma unroll
        for (int k = 0; k < BATCH; ++k) {
            if (p0 + 16 * k >= P) ml[k] = f32x2{NEG_INF, 0.0f};
            mm = fmaxf(mm, ml[k].x);
        }
        if (mm == NEG_INF) continue;
        const float wo = m == NEG_INF ? 0.0f : __expf(m - mm);
        num *= wo;
        den *= wo;
#pragma unroll
        for (int k = 0; k < BATCH; ++k) {
            const float w = ml[k].x == NEG_INF ? 0.0f : __expf(ml[k].x - mm);
            num += ov[k] * w;
            den = fmaf(ml[k].y, w, den);
        }
        m = mm;
    }
    // lanes with equal lane % 4 hold the 16 partition lanes of one column
    float mw = fmaxf(m, dpp_f<0x124>(m));          // row_ror:4
    mw = fmaxf(mw, dpp_f<0x128>(mw));              // row_ror:8
    mw = xmax16(mw);
    const float wt = m == NEG_INF ? 0.0f : __expf(m - mw);
    num *= wt;
    den *= wt;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        num[e] += dpp_f<0x124>(num[e]);
        num[e] = xsum16(num[e] + dpp_f<0x128>(num[e]));
    }
    den += dpp_f<0x124>(den);
    den = xsum16(den + dpp_f<0x128>(den));
    if (lane < 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) iq_store_as(out, sq * out_ss + (int64_t)hq * D + c0 + e, num[e] / den, odt);
    }
}

}  // namespace

static bool valid_block(int64_t B) { return B == 16 || B == 32 || B == 64 || B == 128 || B == 256; }

extern "C" int64_t iq_page_bytes(int64_t H, int64_t block_tokens)
{
    return H * (104 * block_tokens + 832);
}

extern "C" int iq_write_pages(const uint8_t *k_payload, const float *k_scales, const float *k_padding,
                              const void *k_src, const void *k_don, int desc_bytes, const uint8_t *v_payload,
                              const uint16_t *v_scales, const uint16_t *v_offsets, int64_t n_pages, int64_t H,
                              int64_t block_tokens, uint8_t *pool, int64_t pool_pages, const void *page_ids,
                              int id_bytes, void *stream)
{
    IQ_CHECK_ARG(n_pages >= 0 && H >= 1 && H <= 65535, "iq_write_pages: bad shape");
    IQ_CHECK_ARG(valid_block(block_tokens), "iq_write_pages: block_tokens %lld unsupported", (long long)block_tokens);
    IQ_CHECK_ARG(desc_bytes == 1 || desc_bytes == 4 || desc_bytes == 8, "iq_write_pages: desc_bytes");
    IQ_CHECK_ARG(id_bytes == 4 || id_bytes == 8, "iq_write_pages: id_bytes");
    if (n_pages == 0) return IQ_OK;
    IQ_CHECK_ARG(k_payload && k_scales && k_padding && k_src && k_don && v_payload && v_scales && v_offsets &&
                     pool && page_ids, "iq_write_pages: null pointer");
    IQ_CHECK_ARG(n_pages <= 0x7fffffffLL, "iq_write_pages: too many pages");
    IQ_CHECK_ARG(((uintptr_t)k_payload & 15) == 0 && ((uintptr_t)v_payload & 15) == 0 && ((uintptr_t)pool & 15) == 0,
                 "iq_write_pages: payloads and pool must be 16-byte aligned");
    WriteArgs a{k_payload, k_scales, k_padding, k_src, k_don, desc_bytes, v_payload, v_scales, v_offsets, H,
                block_tokens, iq_page_bytes(H, block_tokens), pool_pages, pool, page_ids, id_bytes,
                page_offsets(H, block_tokens)};
    const hipStream_t st = (hipStream_t)stream;
    const bool vec = ((uintptr_t)k_scales & 15) == 0 && ((uintptr_t)k_padding & 15) == 0 &&
                     ((uintptr_t)v_scales & 15) == 0 && ((uintptr_t)v_offsets & 15) == 0;
    if (vec && block_tokens <= 64) {
        const int64_t nph = n_pages * H;
        const dim3 grid((unsigned)((nph + 15) / 16));
        if (block_tokens == 16) hipLaunchKernelGGL((write_small_pages_kernel<16>), grid, dim3(256), 0, st, a, nph);
        else if (block_tokens == 32) hipLaunchKernelGGL((write_small_pages_kernel<32>), grid, dim3(256), 0, st, a, nph);
        else hipLaunchKernelGGL((write_small_pages_kernel<64>), grid, dim3(256), 0, st, a, nph);
        IQ_CHECK_LAUNCH("write_small_pages_kernel");
        return IQ_OK;
    }
    hipLaunchKernelGGL(write_pages_kernel, dim3((unsigned)n_pages, (unsigned)H), dim3(256), 0, st, a);
    IQ_CHECK_LAUNCH("write_pages_kernel");
    return IQ_OK;
}

extern "C" int iq_unpack_pages(const uint8_t *pages, int64_t n_pages, int64_t H, int64_t block_tokens, void *keys,
                               void *values, int out_dtype, void *stream)
{
    IQ_CHECK_ARG(n_pages >= 0 && H >= 1, "iq_unpack_pages: bad shape");
    IQ_CHECK_ARG(valid_block(block_tokens), "iq_unpack_pages: block_tokens %lld unsupported", (long long)block_tokens);
    IQ_CHECK_ARG(out_dtype >= IQ_F32 && out_dtype <= IQ_F16, "iq_unpack_pages: bad out dtype");
    if (n_pages == 0) return IQ_OK;
    IQ_CHECK_ARG(pages && keys && values, "iq_unpack_pages: null pointer");
    IQ_CHECK_ARG(n_pages * H <= 0x7fffffffLL, "iq_unpack_pages: too many pages");
    UnpackArgs a{pages, H, block_tokens, iq_page_bytes(H, block_tokens), page_offsets(H, block_tokens), keys, values,
                 out_dtype};
    const hipStream_t st = (hipStream_t)stream;
    // the row kernels: 16-byte vector stores and loads at page offsets that
    // are multiples of 16 (every supported page size)
    if (((uintptr_t)pages & 15) == 0 && ((uintptr_t)keys & 15) == 0 && ((uintptr_t)values & 15) == 0 &&
        n_pages * H <= 65535) {
        const int64_t nph = n_pages * H;
        if (out_dtype == IQ_BF16) launch_unpack<IQ_BF16>(a, nph, st);
        else if (out_dtype == IQ_F16) launch_unpack<IQ_F16>(a, nph, st);
        else launch_unpack<IQ_F32>(a, nph, st);
        IQ_CHECK_LAUNCH("unpack rows");
        return IQ_OK;
    }
    hipLaunchKernelGGL(unpack_pages_kernel, dim3((unsigned)(n_pages * H), (unsigned)block_tokens), dim3(D), 0, st, a);
    IQ_CHECK_LAUNCH("unpack_pages_kernel");
    return IQ_OK;
}

static int64_t paged_parts(int64_t max_pages, int64_t B)
{
    return (max_pages * B + PART - 1) / PART + (B + 4 + PART - 1) / PART;
}

extern "C" int64_t iq_paged_workspace_floats(int64_t Hq, int64_t n_seq, int64_t max_pages, int64_t block_tokens)
{
    return n_seq * Hq * paged_parts(max_pages, block_tokens) * (D + 2);
}

extern "C" int iq_paged_decode(const void *q, int64_t q_stride_seq, int64_t q_stride_h, int64_t Hq, int64_t n_seq,
                               const uint8_t *pool, int64_t pool_pages, int64_t H, int64_t block_tokens,
                               const int32_t *block_tables, int64_t bt_stride, int64_t max_pages,
                               const int32_t *seq_info, int64_t n_pages, int64_t tail_t, int64_t sink_t,
                               const void *dense, int64_t dense_stride_seq, const int32_t *dense_slots,
                               const int32_t *work, int64_t n_work, float scale, float *workspace,
                               int64_t workspace_floats, void *out, int64_t out_stride_seq, int out_dtype,
                               void *stream)
{
    IQ_CHECK_ARG(q && pool && dense && workspace && out, "iq_paged_decode: null pointer");
    IQ_CHECK_ARG(H >= 1 && Hq >= H && Hq % H == 0 && Hq / H <= 16, "iq_paged_decode: expected 1..16 query heads per KV head");
    IQ_CHECK_ARG(valid_block(block_tokens), "iq_paged_decode: block_tokens %lld unsupported", (long long)block_tokens);
    IQ_CHECK_ARG(n_seq >= 1 && n_seq <= 65535, "iq_paged_decode: bad sequence count");
    IQ_CHECK_ARG(max_pages >= 0 && (max_pages == 0 || block_tables), "iq_paged_decode: missing block table");
    IQ_CHECK_ARG(seq_info || n_seq == 1, "iq_paged_decode: batches need per-sequence lengths");
    IQ_CHECK_ARG(seq_info || (n_pages >= 0 && n_pages <= max_pages && tail_t >= 0 && tail_t <= block_tokens &&
                              sink_t >= 0 && sink_t <= 4), "iq_paged_decode: bad lengths");
    IQ_CHECK_ARG(out_dtype >= IQ_F32 && out_dtype <= IQ_F16, "iq_paged_decode: bad out dtype");
    IQ_CHECK_ARG(((uintptr_t)q & 15) == 0 && q_stride_h % 8 == 0 && q_stride_seq % 8 == 0 &&
                     ((uintptr_t)dense & 15) == 0 && dense_stride_seq % 8 == 0,
                 "iq_paged_decode: query and dense rows must be 16-byte aligned");
    const int64_t parts = paged_parts(max_pages, block_tokens);
    IQ_CHECK_ARG(parts <= 65535, "iq_paged_decode: too many partitions");
    // page fields are addressed with 32-bit offsets from the page
    IQ_CHECK_ARG(iq_page_bytes(H, block_tokens) < (1LL << 32), "iq_paged_decode: pages of 4 GiB or more");
    IQ_CHECK_ARG(workspace_floats >= n_seq * Hq * parts * (D + 2), "iq_paged_decode: workspace too small");
    PagedArgs a{};
    a.q = (const uint16_t *)q;
    a.q_ss = q_stride_seq;
    a.q_sh = q_stride_h;
    a.G = (int)(Hq / H);
    a.H = (int)H;
    a.B = (int)block_tokens;
    a.pool = pool;
    a.page_bytes = iq_page_bytes(H, block_tokens);
    a.pool_pages = pool_pages;
    a.off = page_offsets(H, block_tokens);
    a.bt = block_tables;
    a.bt_ss = bt_stride;
    a.max_pages = max_pages;
    a.seq_info = seq_info;
    a.npg0 = (int)n_pages;
    a.tail0 = (int)tail_t;
    a.sink0 = (int)sink_t;
    a.dense = (const uint16_t *)dense;
    a.dense_ss = dense_stride_seq;
    a.dense_slots = dense_slots;
    a.n_seq = (int)n_seq;
    IQ_CHECK_ARG(!work || (n_work >= 1 && n_work <= 65535 && n_seq <= 32767),
                 "iq_paged_decode: the work list holds 1 to 65535 items of at most 32767 sequences");
    a.work = work;
    a.max_parts = (int)parts;
    a.c_log2 = scale * 1.4426950408889634f;
    a.ws = workspace;
    const dim3 grid((unsigned)H, (unsigned)(a.work ? n_work : parts), (unsigned)(a.work ? 1 : n_seq));
    hipStream_t st = (hipStream_t)stream;
    switch (block_tokens) {
    case 16: hipLaunchKernelGGL(decode_paged<16>, grid, dim3(256), 0, st, a); break;
    case 32: hipLaunchKernelGGL(decode_paged<8>, grid, dim3(256), 0, st, a); break;
    case 64: hipLaunchKernelGGL(decode_paged<4>, grid, dim3(256), 0, st, a); break;
    case 128: hipLaunchKernelGGL(decode_paged<2>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(decode_paged<1>, grid, dim3(256), 0, st, a); break;
    }
    IQ_CHECK_LAUNCH("decode_paged");
    hipLaunchKernelGGL(paged_reduce, dim3((unsigned)(64 * ((Hq + 7) / 8)), 1, (unsigned)n_seq), dim3(64), 0, st, a, out,
                       out_stride_seq, out_dtype);
    IQ_CHECK_LAUNCH("paged_reduce");
    return IQ_OK;
}
