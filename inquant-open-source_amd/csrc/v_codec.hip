// Group-wise affine value codec (V2 / V4) and the K4/V dequantizers (gfx950).
//
// Encode (value_codec.py:51-72), per (token, group of `group` channels):
//   lo = min, hi = max;  offset = f16(lo);
//   scale = f16(max((hi - lo) / levels, 2^-14));
//   code = clamp(rint((x - f32(offset)) / f32(scale)), 0, levels);
//   codes packed LSB-first, 8/bits per byte.
// Decode (value_codec.py:38-48): code * f32(scale) + f32(offset).  The
// product of a <=4-bit code and an f16 scale is exact in fp32, so the
// reference's separate multiply and add round exactly once.
#include "v_rows_dev.h"

namespace {

constexpr int V_THREADS = 256;

struct VEncArgs {
    const void *x;
    int dt;
    int64_t sb, sh, st, sc;
    int64_t H, T, D;
    int bits, group;
    int64_t units;          // B*H*T*(D/8): eight channels of one token each
    int vec;                // rows are channel-contiguous and 16-byte aligned
    uint8_t *payload;
    uint16_t *scales, *offsets;
    int *bad;
};

// Eight consecutive channels of x as fp32.
__device__ __forceinline__ void v_load8(const VEncArgs &a, int64_t base, float v[8])
{
    if (a.vec && (a.dt == IQ_BF16 || a.dt == IQ_F16)) {
        const u32x4_t r = *(const u32x4_t *)((const uint16_t *)a.x + base);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t h = (uint16_t)(r[e >> 1] >> (16 * (e & 1)));
            v[e] = a.dt == IQ_F16 ? iq_f16_to_f32(h) : iq_bf16_to_f32(h);
        }
    } else if (a.vec && a.dt == IQ_F32) {
        const u32x4_t r0 = *(const u32x4_t *)((const float *)a.x + base);
        const u32x4_t r1 = *(const u32x4_t *)((const float *)a.x + base + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = __uint_as_float(r0[e]);
            v[4 + e] = __uint_as_float(r1[e]);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = iq_load_f32(a.x, base + e * a.sc, a.dt);
    }
}

// One thread per eight channels of one token; the group/8 lanes of a group
// reduce min and max with cross-lane exchanges and the group's first lane
// writes its f16 scale and offset.
__global__ __launch_bounds__(V_THREADS) void v_encode_kernel(VEncArgs a)
{
    const int64_t u = (int64_t)blockIdx.x * V_THREADS + threadIdx.x;
    const bool live = u < a.units;
    const int64_t per_row = a.D / 8;
    const int64_t r = live ? u / per_row : 0, j = live ? u - r * per_row : 0;   // r = (b*H + h)*T + t
    const int64_t t = r % a.T, bh = r / a.T;
    const int64_t b = bh / a.H, h = bh % a.H;
    const int64_t base = b * a.sb + h * a.sh + t * a.st + 8 * j * a.sc;
    const int levels = (1 << a.bits) - 1;
    const int lanes = a.group / 8;

    float v[8];
    if (live) v_load8(a, base, v);
    else
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    bool bad = false;
    float lo = v[0], hi = v[0];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        bad |= !iq_isfinite(v[e]);
        lo = fminf(lo, v[e]);
        hi = fmaxf(hi, v[e]);
    }
    for (int o = 1; o < lanes; o <<= 1) {
        lo = fminf(lo, __shfl_xor(lo, o, 64));
        hi = fmaxf(hi, __shfl_xor(hi, o, 64));
    }
    const uint16_t off_h = iq_f32_to_f16(lo);
    float s = __fsub_rn(hi, lo) / (float)levels;
    const float tiny = 6.103515625e-05f;
    s = s < tiny ? tiny : s;
    const uint16_t sc_h = iq_f32_to_f16(s);
    const float off = iq_f16_to_f32(off_h), sc = iq_f16_to_f32(sc_h);
    bad |= !iq_isfinite(off) || !iq_isfinite(sc);

    const float rsc = __builtin_amdgcn_rcpf(sc);
    float d[8], q[8];
    bool near = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        d[e] = __fsub_rn(v[e], off);
        const float f = __fmul_rn(d[e], rsc);
        q[e] = rintf(f);
        near |= !(0.5f - fabsf(__fsub_rn(f, q[e])) > fabsf(f) * 0x1p-20f);
    }
    if (near) {            // a quotient near a rounding boundary: exact division decides
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = iq_rint_div(d[e], sc, rsc);
    }
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) word |= (uint32_t)fminf(fmaxf(q[e], 0.0f), (float)levels) << (e * a.bits);
    if (live) {
        if (j % lanes == 0) {
            const int64_t gi = r * (a.D / a.group) + j / lanes;
            a.offsets[gi] = off_h;
            a.scales[gi] = sc_h;
        }
        if (a.bits == 2) ((uint16_t *)a.payload)[u] = (uint16_t)word;
        else ((uint32_t *)a.payload)[u] = word;
    }
    if (__ballot(live && bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(a.bad, 1);
}

// Rows of 16-bit values with unit channel stride and 16-byte aligned rows,
// D = 16 * PR channels.  Grid (token blocks, B*H); each thread encodes 16
// consecutive channels of NT tokens with v_encode16 (v_rows_dev.h), GL =
// group / 16 adjacent lanes forming one group: the same codes as
// v_encode_kernel with fewer instructions.
struct VRowArgs {
    const uint16_t *x;
    int64_t sb, sh, st;      // element strides of batch, head, token
    int H, T;
    uint8_t *payload;
    uint16_t *scales, *offsets;
    int *bad;
};

template <bool F16IN, int BITS, int GL, int PR, int NT>
__global__ __launch_bounds__(V_THREADS) void v_encode_rows(VRowArgs a)
{
    constexpr int TPB = V_THREADS / PR;                   // tokens per pass of the block
    constexpr int D = 16 * PR, GROUPS = PR / GL;          // groups per token
    constexpr int PB = D * BITS / 8;                      // payload bytes per token
    const int tid = threadIdx.x;
    const int j = tid % PR, tl = tid / PR;
    const int bh = blockIdx.y, b = bh / a.H, h = bh - b * a.H;
    const int t0 = blockIdx.x * (TPB * NT);
    const uint16_t *xb = a.x + b * a.sb + h * a.sh + (int64_t)t0 * a.st + 16 * j;
    const int64_t r0 = (int64_t)bh * a.T + t0;            // first row of the block

    u32x4_t raw[NT][2];
#pragma unroll
    for (int k = 0; k < NT; ++k) {
        const int tk = min(tl + k * TPB, a.T - 1 - t0);   // clamp the tail to the last token
        const u32x4_t *p = (const u32x4_t *)(xb + (uint32_t)tk * (uint32_t)a.st);
        raw[k][0] = __builtin_nontemporal_load(p);
        raw[k][1] = __builtin_nontemporal_load(p + 1);
    }
    bool bad = false;
#pragma unroll
    for (int k = 0; k < NT; ++k) {
        const int tk = tl + k * TPB;
        const bool live = t0 + tk < a.T;
        uint32_t word[BITS / 2];
        uint16_t off_h, sc_h;
        v_encode16<F16IN, BITS, GL>(raw[k], live, word, off_h, sc_h, bad);
        const int row = tk;   // row offset within the block
        if (live) {
            if (BITS == 2) {
                __builtin_nontemporal_store(word[0], (uint32_t *)(a.payload + r0 * PB + (uint32_t)(row * PB + 4 * j)));
            } else {
                typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;
                *(u32x2_t *)(a.payload + r0 * PB + (uint32_t)(row * PB + 8 * j)) = u32x2_t{word[0], word[BITS / 2 - 1]};
            }
            const int64_t gi = r0 * GROUPS + (uint32_t)(row * GROUPS + j / GL);
            if (j % GL == 0) a.offsets[gi] = off_h;
            if (j % GL == GL - 1) a.scales[gi] = sc_h;
        }
    }
    if (__ballot(bad) != 0 && (tid & 63) == 0) atomicOr(a.bad, 1);
}

template <bool F16IN, int BITS, int GL>
bool v_rows_dispatch_pr(int PR, dim3 grid, hipStream_t st, const VRowArgs &a)
{
    switch (PR) {
#define IQ_V_CASE(P)                                                                              \
    case P:                                                                                       \
        if constexpr (GL <= P) {                                                                  \
            hipLaunchKernelGGL((v_encode_rows<F16IN, BITS, GL, P, 2>), grid, dim3(V_THREADS), 0, st, a); \
            return true;                                                                          \
        }                                                                                         \
        return false;
    IQ_V_CASE(2)
    IQ_V_CASE(4)
    IQ_V_CASE(8)
    IQ_V_CASE(16)
#undef IQ_V_CASE
    default: return false;
    }
}

template <bool F16IN, int BITS>
bool v_rows_dispatch_gl(int GL, int PR, dim3 grid, hipStream_t st, const VRowArgs &a)
{
    switch (GL) {
    case 2: return v_rows_dispatch_pr<F16IN, BITS, 2>(PR, grid, st, a);
    case 4: return v_rows_dispatch_pr<F16IN, BITS, 4>(PR, grid, st, a);
    case 8: return v_rows_dispatch_pr<F16IN, BITS, 8>(PR, grid, st, a);
    default: return false;
    }
}

struct VDecArgs {
    const uint8_t *payload;
    const uint16_t *scales, *offsets;
    int64_t rows, D;
    int bits, group;
    void *out;
    int out_dt;
};

__global__ __launch_bounds__(V_THREADS) void v_decode_kernel(VDecArgs a)
{
    const int64_t i = (int64_t)blockIdx.x * V_THREADS + threadIdx.x;
    if (i >= a.rows * a.D) return;
    const int64_t r = i / a.D, c = i - r * a.D;
    const int per_byte = 8 / a.bits;
    const int code = (a.payload[r * (a.D / per_byte) + c / per_byte] >> ((c % per_byte) * a.bits)) &
                     ((1 << a.bits) - 1);
    const int64_t p = r * (a.D / a.group) + c / a.group;
    const float v = __fadd_rn(__fmul_rn((float)code, iq_f16_to_f32(a.scales[p])), iq_f16_to_f32(a.offsets[p]));
    iq_store_as(a.out, i, v, a.out_dt);
}

struct KDecArgs {
    const uint8_t *payload;
    const float *scales;
    const void *src, *don;
    int desc_bytes;
    const float *padding;
    int64_t rows, T, D, count;
    void *out;
    int out_dt;
};

__device__ __forceinline__ int load_desc(const void *p, int64_t i, int bytes)
{
    if (bytes == 1) return ((const uint8_t *)p)[i];
    if (bytes == 4) return ((const int32_t *)p)[i];
    return (int)((const int64_t *)p)[i];
}

// One workgroup per (row, token); roles are rebuilt per workgroup in LDS.
__global__ __launch_bounds__(V_THREADS) void k4_decode_kernel(KDecArgs a)
{
    __shared__ int16_t s_role[1024];
    const int64_t rt = blockIdx.x;            // row * T + t
    const int64_t row = rt / a.T;
    for (int64_t c = threadIdx.x; c < a.D; c += V_THREADS) s_role[c] = -1;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < a.count; i += V_THREADS) {
        const int s = load_desc(a.src, row * a.count + i, a.desc_bytes);
        const int d = load_desc(a.don, row * a.count + i, a.desc_bytes);
        s_role[s] = (int16_t)d;
        s_role[d] = (int16_t)(-2 - i);
    }
    __syncthreads();
    const uint8_t *pt = a.payload + rt * (a.D / 2);
    for (int64_t c = threadIdx.x; c < a.D; c += V_THREADS) {
        const int role = s_role[c];
        const int slot = (pt[c >> 1] >> ((c & 1) * 4)) & 15;
        float v;
        if (role >= 0) {
            const int lo = (pt[role >> 1] >> ((role & 1) * 4)) & 15;
            v = __fmul_rn((float)(((slot << 4) | lo) - 128), a.scales[row * a.D + c]);
        } else if (role <= -2) {
            v = a.padding[row * a.count + (-role - 2)];
        } else {
            v = __fmul_rn((float)(slot - 8), a.scales[row * a.D + c]);
        }
        iq_store_as(a.out, rt * a.D + c, v, a.out_dt);
    }
}

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_nt;

// Two values rounded to the 16-bit output dtype (nearest even), first in
// the low half: one conversion instruction for the pair.
template <int OUT>
__device__ __forceinline__ uint32_t pack_pair(float x, float y)
{
    if constexpr (OUT == IQ_BF16) {
        typedef __attribute__((ext_vector_type(2))) __bf16 pair_t;
        return __builtin_bit_cast(uint32_t, pair_t{(__bf16)x, (__bf16)y});
    } else {
        typedef __attribute__((ext_vector_type(2))) _Float16 pair_t;
        return __builtin_bit_cast(uint32_t, pair_t{(_Float16)x, (_Float16)y});
    }
}

// Rows of 128 channels, 16-byte aligned output rows.  Thread (row, j)
// decodes channels 16 j .. 16 j + 15 of one row: BITS / 2 payload words and
// its group's f16 scale and offset, then writes 16 values with 16-byte
// stores.  Same arithmetic as v_decode_kernel.
template <int BITS, int OUT>
__global__ __launch_bounds__(V_THREADS) void v_decode_rows(VDecArgs a)
{
    const int64_t u = (int64_t)blockIdx.x * V_THREADS + threadIdx.x;
    const int64_t r = u >> 3;
    const int j = (int)(u & 7);
    if (r >= a.rows) return;
    constexpr int PB = 128 * BITS / 8;                      // payload bytes per row
    const int64_t p = r * (128 / a.group) + (16 * j) / a.group;
    const float sc = iq_f16_to_f32(a.scales[p]), off = iq_f16_to_f32(a.offsets[p]);
    uint64_t w;                                             // channel 16 j + e at bits BITS * e
    if constexpr (BITS == 2) w = *(const uint32_t *)(a.payload + r * PB + 4 * j);
    else w = *(const uint64_t *)(a.payload + r * PB + 8 * j);
    float v[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int code = (int)((w >> (BITS * e)) & ((1u << BITS) - 1u));
        v[e] = __fadd_rn(__fmul_rn((float)code, sc), off);
    }
    if constexpr (OUT == IQ_F32) {
        float4 *o = (float4 *)((float *)a.out + r * 128 + 16 * j);
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = float4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
    } else {
        uint32_t h[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) h[k] = pack_pair<OUT>(v[2 * k], v[2 * k + 1]);
        u32x4_nt *o = (u32x4_nt *)((uint16_t *)a.out + r * 128 + 16 * j);
        __builtin_nontemporal_store(u32x4_nt{h[0], h[1], h[2], h[3]}, o);
        __builtin_nontemporal_store(u32x4_nt{h[4], h[5], h[6], h[7]}, o + 1);
    }
}

// Blocks of 128 channels with at most 64 one-byte descriptors, 16-byte
// aligned output rows.  Grid (token tiles of 128, rows); the row's role map,
// scales and donor paddings are built once in LDS.  Thread (token, j),
// j < 16, decodes channels 8 j .. 8 j + 7 of a token from one payload word;
// a source channel's low nibble comes from the donor's word, read from the
// lane of the token that holds it.  Same arithmetic as k4_decode_kernel.
// The thread's KD_ITER payload words are loaded first, before the role
// tables are built, so one memory round trip covers them all.
constexpr int KD_TOKENS = 128;
constexpr int KD_ITER = KD_TOKENS / (V_THREADS / 16);   // tokens per thread

template <int OUT>
__global__ __launch_bounds__(V_THREADS) void k4_decode_rows(KDecArgs a)
{
    __shared__ float s_scale[128], s_pad[64];
    __shared__ int16_t s_role[128];
    const int tid = threadIdx.x, lane = tid & 63;
    const int64_t row = blockIdx.y;
    const int j = tid & 15;
    const int64_t t_first = (int64_t)blockIdx.x * KD_TOKENS + (tid >> 4);
    uint32_t words[KD_ITER];
#pragma unroll
    for (int i = 0; i < KD_ITER; ++i) {
        const int64_t t = t_first + i * (V_THREADS / 16);
        const int64_t rt = row * a.T + (t < a.T ? t : a.T - 1);   // every lane loads (the shuffles need all)
        words[i] = *(const uint32_t *)(a.payload + rt * 64 + 4 * j);
    }
    if (tid < 128) {
        s_scale[tid] = a.scales[row * 128 + tid];
        s_role[tid] = -1;
    }
    __syncthreads();
    if (tid < a.count) {
        const int sch = ((const uint8_t *)a.src)[row * a.count + tid];
        const int dch = ((const uint8_t *)a.don)[row * a.count + tid];
        if (sch < 128 && dch < 128) {
            s_role[sch] = (int16_t)dch;
            s_role[dch] = (int16_t)(-2 - tid);
        }
        s_pad[tid] = a.padding[row * a.count + tid];
    }
    __syncthreads();
    // per slot e of this lane (channel 8 j + e), fixed across tokens: the
    // value is code * f with code = slot * m + lo - off: a plain channel has
    // m = 1, off = 8, f its scale; a source m = 16, off = 128, f its scale
    // and lo its donor's nibble; a donor m = 0, off = -1 (code 1) and f its
    // padding, so every slot is one product and no lane branches.  lo is a
    // zero-width field extract except at a source; a donor outside this
    // lane's word comes from the lane of its 16 that holds it (the eight
    // cross-lane reads of a token are issued together)
    uint32_t m[8], lo_at[8], lo_w[8];
    int off[8], bp[8];
    bool xl[8];
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int rl = s_role[8 * j + e];
        const bool src = rl >= 0, don = rl <= -2;
        f[e] = don ? s_pad[-rl - 2] : s_scale[8 * j + e];
        m[e] = src ? 16u : don ? 0u : 1u;
        off[e] = src ? 128 : don ? -1 : 8;
        lo_w[e] = src ? 4u : 0u;
        lo_at[e] = src ? 4u * (uint32_t)(rl & 7) : 0u;
        xl[e] = src && (rl >> 3) != j;
        bp[e] = 4 * ((lane & ~15) | ((rl >> 3) & 15));       // ds_bpermute address of word rl / 8
    }
#pragma unroll
    for (int i = 0; i < KD_ITER; ++i) {
        const int64_t t = t_first + i * (V_THREADS / 16);
        const bool live = t < a.T;
        const int64_t rt = row * a.T + (live ? t : a.T - 1);
        const uint32_t w = words[i];
        uint32_t x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (uint32_t)__builtin_amdgcn_ds_bpermute(bp[e], (int)w);
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t wd = xl[e] ? x[e] : w;
            const uint32_t slot = __builtin_amdgcn_ubfe(w, 4 * e, 4);
            const uint32_t lo = __builtin_amdgcn_ubfe(wd, lo_at[e], lo_w[e]);
            const int code = (int)(__umul24(slot, m[e]) + lo) - off[e];
            v[e] = __fmul_rn((float)code, f[e]);
        }
        if (!live) continue;
        if constexpr (OUT == IQ_F32) {
            float4 *o = (float4 *)((float *)a.out + rt * 128 + 8 * j);
            o[0] = float4{v[0], v[1], v[2], v[3]};
            o[1] = float4{v[4], v[5], v[6], v[7]};
        } else {
            uint32_t h[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) h[k] = pack_pair<OUT>(v[2 * k], v[2 * k + 1]);
            __builtin_nontemporal_store(u32x4_nt{h[0], h[1], h[2], h[3]}, (u32x4_nt *)((uint16_t *)a.out + rt * 128 + 8 * j));
        }
    }
}

}  // namespace

extern "C" int iq_v_quantize(const void *x, int x_dtype, const int64_t *x_strides, int64_t B, int64_t H,
                             int64_t T, int64_t D, int bits, int group, uint8_t *payload, uint16_t *scales,
                             uint16_t *offsets, int *bad_flag, void *stream)
{
    IQ_CHECK_ARG(x && x_strides && payload && scales && offsets && bad_flag, "iq_v_quantize: null pointer");
    IQ_CHECK_ARG(x_dtype >= IQ_F32 && x_dtype <= IQ_F64, "iq_v_quantize: bad dtype");
    IQ_CHECK_ARG(bits == 2 || bits == 4, "iq_v_quantize: bits must be 2 or 4");
    IQ_CHECK_ARG(group == 32 || group == 64 || group == 128, "iq_v_quantize: group must be 32, 64 or 128");
    IQ_CHECK_ARG(B >= 1 && H >= 1 && T >= 1 && D >= group && D % group == 0, "iq_v_quantize: bad shape");
    const int64_t units = B * H * T * (D / 8);
    IQ_CHECK_ARG((units + V_THREADS - 1) / V_THREADS <= 0x7fffffffLL, "iq_v_quantize: too large");
    const int64_t elt = x_dtype == IQ_F32 ? 4 : x_dtype == IQ_F64 ? 8 : 2;
    const int64_t vmul = 16 / elt;         // elements per 16 bytes
    const int vec = x_dtype != IQ_F64 && x_strides[3] == 1 && x_strides[0] % vmul == 0 &&
                    x_strides[1] % vmul == 0 && x_strides[2] % vmul == 0 && ((uintptr_t)x & 15) == 0;
    const int64_t PR = D / 16;
    if (vec && (x_dtype == IQ_BF16 || x_dtype == IQ_F16) && D % 16 == 0 && (PR == 2 || PR == 4 || PR == 8 || PR == 16) &&
        B * H <= 65535 && T <= 0x7fffffffLL - 512 && x_strides[2] >= 0 && x_strides[2] <= (1 << 23)) {
        const int64_t span = (V_THREADS / PR) * 2;          // tokens per block
        const dim3 grid((unsigned)((T + span - 1) / span), (unsigned)(B * H));
        const VRowArgs ra{(const uint16_t *)x, x_strides[0], x_strides[1], x_strides[2], (int)H, (int)T,
                          payload, scales, offsets, bad_flag};
        const int GL = group / 16;
        const hipStream_t st = (hipStream_t)stream;
        const bool ok = x_dtype == IQ_F16
                            ? (bits == 2 ? v_rows_dispatch_gl<true, 2>(GL, (int)PR, grid, st, ra)
                                         : v_rows_dispatch_gl<true, 4>(GL, (int)PR, grid, st, ra))
                            : (bits == 2 ? v_rows_dispatch_gl<false, 2>(GL, (int)PR, grid, st, ra)
                                         : v_rows_dispatch_gl<false, 4>(GL, (int)PR, grid, st, ra));
        if (ok) {
            IQ_CHECK_LAUNCH("v_encode_rows");
            return IQ_OK;
        }
    }
    VEncArgs a{x, x_dtype, x_strides[0], x_strides[1], x_strides[2], x_strides[3], H, T, D, bits, group, units,
               vec, payload, scales, offsets, bad_flag};
    hipLaunchKernelGGL(v_encode_kernel, dim3((unsigned)((units + V_THREADS - 1) / V_THREADS)), dim3(V_THREADS), 0,
                       (hipStream_t)stream, a);
    IQ_CHECK_LAUNCH("v_encode_kernel");
    return IQ_OK;
}

extern "C" int iq_v_dequantize(const uint8_t *payload, const uint16_t *scales, const uint16_t *offsets,
                               int64_t rows, int64_t D, int bits, int group, void *out, int out_dtype, void *stream)
{
    IQ_CHECK_ARG(bits == 2 || bits == 4, "iq_v_dequantize: bits must be 2 or 4");
    IQ_CHECK_ARG(group == 32 || group == 64 || group == 128, "iq_v_dequantize: bad group");
    IQ_CHECK_ARG(rows >= 0 && D >= group && D % group == 0, "iq_v_dequantize: bad shape");
    IQ_CHECK_ARG(out_dtype >= IQ_F32 && out_dtype <= IQ_F16, "iq_v_dequantize: bad out dtype");
    if (rows == 0) return IQ_OK;
    IQ_CHECK_ARG(payload && scales && offsets && out, "iq_v_dequantize: null pointer");
    const int64_t n = rows * D;
    VDecArgs a{payload, scales, offsets, rows, D, bits, group, out, out_dtype};
    if (D == 128 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)payload & (bits == 2 ? 3 : 7)) == 0 &&
        (rows * 8 + V_THREADS - 1) / V_THREADS <= 0x7fffffffLL) {
        const dim3 grid((unsigned)((rows * 8 + V_THREADS - 1) / V_THREADS)), block(V_THREADS);
        const hipStream_t st = (hipStream_t)stream;
        if (bits == 2) {
            if (out_dtype == IQ_BF16) hipLaunchKernelGGL((v_decode_rows<2, IQ_BF16>), grid, block, 0, st, a);
            else if (out_dtype == IQ_F16) hipLaunchKernelGGL((v_decode_rows<2, IQ_F16>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((v_decode_rows<2, IQ_F32>), grid, block, 0, st, a);
        } else {
            if (out_dtype == IQ_BF16) hipLaunchKernelGGL((v_decode_rows<4, IQ_BF16>), grid, block, 0, st, a);
            else if (out_dtype == IQ_F16) hipLaunchKernelGGL((v_decode_rows<4, IQ_F16>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((v_decode_rows<4, IQ_F32>), grid, block, 0, st, a);
        }
        IQ_CHECK_LAUNCH("v_decode_rows");
        return IQ_OK;
    }
    hipLaunchKernelGGL(v_decode_kernel, dim3((unsigned)((n + V_THREADS - 1) / V_THREADS)), dim3(V_THREADS), 0,
                       (hipStream_t)stream, a);
    IQ_CHECK_LAUNCH("v_decode_kernel");
    return IQ_OK;
}

extern "C" int iq_k4_dequantize(const uint8_t *payload, const float *scales, const void *src, const void *don,
                                int desc_bytes, const float *padding, int64_t rows, int64_t T, int64_t D,
                                int64_t count, void *out, int out_dtype, void *stream)
{
    IQ_CHECK_ARG(D >= 2 && D % 2 == 0 && D <= 1024, "iq_k4_dequantize: bad D");
    IQ_CHECK_ARG(count >= 0 && 2 * count <= D, "iq_k4_dequantize: bad count");
    IQ_CHECK_ARG(desc_bytes == 1 || desc_bytes == 4 || desc_bytes == 8, "iq_k4_dequantize: desc_bytes");
    IQ_CHECK_ARG(out_dtype >= IQ_F32 && out_dtype <= IQ_F16, "iq_k4_dequantize: bad out dtype");
    IQ_CHECK_ARG(rows >= 0 && T >= 0, "iq_k4_dequantize: bad shape");
    if (rows == 0 || T == 0) return IQ_OK;
    IQ_CHECK_ARG(payload && scales && out && (count == 0 || (src && don && padding)), "iq_k4_dequantize: null");
    IQ_CHECK_ARG(rows * T <= 0x7fffffffLL, "iq_k4_dequantize: too large");
    KDecArgs a{payload, scales, src, don, desc_bytes, padding, rows, T, D, count, out, out_dtype};
    if (D == 128 && desc_bytes == 1 && count <= 64 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)payload & 3) == 0 &&
        rows <= 65535 && out_dtype != IQ_F64) {
        const dim3 grid((unsigned)((T + KD_TOKENS - 1) / KD_TOKENS), (unsigned)rows), block(V_THREADS);
        const hipStream_t st = (hipStream_t)stream;
        if (out_dtype == IQ_BF16) hipLaunchKernelGGL((k4_decode_rows<IQ_BF16>), grid, block, 0, st, a);
        else if (out_dtype == IQ_F16) hipLaunchKernelGGL((k4_decode_rows<IQ_F16>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((k4_decode_rows<IQ_F32>), grid, block, 0, st, a);
        IQ_CHECK_LAUNCH("k4_decode_rows");
        return IQ_OK;
    }
    hipLaunchKernelGGL(k4_decode_kernel, dim3((unsigned)(rows * T)), dim3(V_THREADS), 0, (hipStream_t)stream, a);
    IQ_CHECK_LAUNCH("k4_decode_kernel");
    return IQ_OK;
}
