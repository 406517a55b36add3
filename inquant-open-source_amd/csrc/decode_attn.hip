// Fused single-query GQA decode attention over [sink | packed blocks | tail].
//
// Semantics follow PackedDecodeState.decode (triton_attention.py:317-388):
// one partition per packed block and per 32-token slice of the dense
// sink and tail; keys and values are decoded from the K4 / V2 / V4 formats
// (_decode_tile :33-50, _decode_value_tile :53-64), rounded to the query
// dtype exactly as the dequantize-then-attend path does, and each
// partition's (acc[128], m, l) online-softmax partial is merged by a
// log-sum-exp reduction (_reduce_partials :168-181).  Softmax weights stay
// in fp32 for the P.V product.
//
// This file holds the general kernel (any query dtype, K4- or V2/V4-coded
// values, G <= 16 query heads per KV head, VALU arithmetic).
#include <mutex>

#include "decode_common.h"

namespace {

constexpr int DA_THREADS = 256;
constexpr int TILE = 32;
constexpr int D = 128;
constexpr int GMAX = 16;
constexpr int DENSE_SPLIT = 32;     // as the matrix-core path, so one workspace size covers both

struct DecodeArgs {
    const void *q;
    int qdt;
    int64_t q_sh, Hq;
    const int64_t *tables;
    const int8_t *kmap, *vmap;
    int64_t nblk, BT, H, S;
    int vbits, vgroup;
    const void *sk, *sv;
    int64_t sk_sh, sk_st, sv_sh, sv_st, sink_t;
    const void *tk, *tv;
    int64_t tk_sh, tk_st, tv_sh, tv_st, tail_t;
    float scale;
    float *ws;
    int64_t P;
    int G;
    void *out;
    int odt;
};

// K4 element: role >= 0 source (partner = role), role <= -2 donor, -1 normal.
__device__ __forceinline__ float k4_element(const uint8_t *row, const float *scales, const float *padding,
                                            int role, int c)
{
    const int slot = (row[c >> 1] >> ((c & 1) * 4)) & 15;
    if (role >= 0) {
        const int lo = (row[role >> 1] >> ((role & 1) * 4)) & 15;
        return __fmul_rn((float)(((slot << 4) | lo) - 128), scales[c]);
    }
    if (role <= -2) return padding[-role - 2];
    return __fmul_rn((float)(slot - 8), scales[c]);
}

__global__ __launch_bounds__(DA_THREADS) void decode_partials_generic(DecodeArgs a)
{
    __shared__ float s_q[GMAX][D];
    __shared__ float s_k[TILE][D + 1];
    __shared__ float s_v[TILE][D];
    __shared__ float s_p[GMAX][TILE];
    __shared__ float s_m[GMAX], s_l[GMAX], s_alpha[GMAX];
    __shared__ int8_t s_krole[D], s_vrole[D];
    __shared__ float s_kscale[D], s_vscale[D];
    __shared__ float s_kpad[64], s_vpad[64];

    const int tid = threadIdx.x;
    const int h = blockIdx.x;
    const int64_t p = blockIdx.y;
    const int G = a.G;

    for (int i = tid; i < GMAX * D; i += DA_THREADS) {
        const int g = i / D, d = i % D;
        s_q[g][d] = g < G ? iq_load_f32(a.q, (int64_t)(h * G + g) * a.q_sh + d, a.qdt) : 0.0f;
    }
    if (tid < GMAX) {
        s_m[tid] = -__uint_as_float(0x7f800000u);
        s_l[tid] = 0.0f;
    }

    // Partition geometry.
    const bool packed = p < a.nblk;
    const uint8_t *kpay = nullptr, *vpay = nullptr;
    const uint16_t *vsc16 = nullptr, *voff16 = nullptr;
    const void *dk = nullptr, *dv = nullptr;
    int64_t dk_sh = 0, dk_st = 0, dv_sh = 0, dv_st = 0, start = 0, length = 0;
    if (packed) {
        const int64_t *row = a.tables + p * IQ_TABLE_COLS;
        kpay = (const uint8_t *)row[0] + (int64_t)h * a.BT * (D / 2);
        const float *ksc = (const float *)row[1] + h * D;
        const float *kpad = (const float *)row[2] + h * a.S;
        vpay = (const uint8_t *)row[3];
        for (int c = tid; c < D; c += DA_THREADS) {
            s_krole[c] = a.kmap[(p * a.H + h) * D + c];
            s_kscale[c] = ksc[c];
        }
        for (int i = tid; i < a.S; i += DA_THREADS) s_kpad[i] = kpad[i];
        if (a.vbits == 0) {
            vpay += (int64_t)h * a.BT * (D / 2);
            const float *vsc = (const float *)row[4] + h * D;
            const float *vpad = (const float *)row[5] + h * a.S;
            for (int c = tid; c < D; c += DA_THREADS) {
                s_vrole[c] = a.vmap[(p * a.H + h) * D + c];
                s_vscale[c] = vsc[c];
            }
            for (int i = tid; i < a.S; i += DA_THREADS) s_vpad[i] = vpad[i];
        } else {
            vsc16 = (const uint16_t *)row[4];
            voff16 = (const uint16_t *)row[5];
        }
        start = 0;
        length = a.BT;
    } else {
        const int64_t dp = p - a.nblk;
        const int64_t sink_parts = (a.sink_t + DENSE_SPLIT - 1) / DENSE_SPLIT;
        if (dp < sink_parts) {
            dk = a.sk; dv = a.sv;
            dk_sh = a.sk_sh; dk_st = a.sk_st; dv_sh = a.sv_sh; dv_st = a.sv_st;
            start = dp * DENSE_SPLIT;
            length = a.sink_t;
        } else {
            dk = a.tk; dv = a.tv;
            dk_sh = a.tk_sh; dk_st = a.tk_st; dv_sh = a.tv_sh; dv_st = a.tv_st;
            start = (dp - sink_parts) * DENSE_SPLIT;
            length = a.tail_t;
        }
    }
    const int64_t stop = packed ? a.BT : (start + DENSE_SPLIT < length ? start + DENSE_SPLIT : length);
    __syncthreads();

    // Accumulators: thread owns channel d and query rows g0, g0 + 2, ...
    const int d = tid % D;
    const int g0 = tid / D;
    float acc[GMAX / 2];
#pragma unroll
    for (int k = 0; k < GMAX / 2; ++k) acc[k] = 0.0f;

    for (int64_t base = start; base < stop; base += TILE) {
        // decode K and V tiles (rounded to the query dtype)
        for (int i = tid; i < TILE * D; i += DA_THREADS) {
            const int t = i / D, c = i % D;
            const int64_t tok = base + t;
            float kv = 0.0f, vv = 0.0f;
            if (tok < stop) {
                if (packed) {
                    kv = k4_element(kpay + tok * (D / 2), s_kscale, s_kpad, s_krole[c], c);
                    if (a.vbits == 0) {
                        vv = k4_element(vpay + tok * (D / 2), s_vscale, s_vpad, s_vrole[c], c);
                    } else {
                        const int per_byte = 8 / a.vbits;
                        const int64_t vr = (int64_t)h * a.BT + tok;
                        const int code = (vpay[vr * (D / per_byte) + c / per_byte] >> ((c % per_byte) * a.vbits)) &
                                         ((1 << a.vbits) - 1);
                        const int64_t pi = vr * (D / a.vgroup) + c / a.vgroup;
                        vv = __fadd_rn(__fmul_rn((float)code, iq_f16_to_f32(vsc16[pi])), iq_f16_to_f32(voff16[pi]));
                    }
                    kv = iq_round_to(kv, a.qdt);
                    vv = iq_round_to(vv, a.qdt);
                } else {
                    kv = iq_load_f32(dk, h * dk_sh + tok * dk_st + c, a.qdt);
                    vv = iq_load_f32(dv, h * dv_sh + tok * dv_st + c, a.qdt);
                }
            }
            s_k[t][c] = kv;
            s_v[t][c] = vv;
        }
        __syncthreads();
        // logits
        for (int i = tid; i < GMAX * TILE; i += DA_THREADS) {
            const int g = i / TILE, t = i % TILE;
            float s = -__uint_as_float(0x7f800000u);
            if (g < G && base + t < stop) {
                float dot = 0.0f;
                for (int c = 0; c < D; ++c) dot = fmaf(s_q[g][c], s_k[t][c], dot);
                s = dot * a.scale;
            }
            s_p[g][t] = s;
        }
        __syncthreads();
        // online softmax, one thread per query row
        if (tid < G) {
            const int g = tid;
            float mx = s_m[g];
            for (int t = 0; t < TILE; ++t) mx = fmaxf(mx, s_p[g][t]);
            const float alpha = expf(s_m[g] - mx);
            float sum = 0.0f;
            for (int t = 0; t < TILE; ++t) {
                const float e = expf(s_p[g][t] - mx);
                s_p[g][t] = e;
                sum += e;
            }
            s_l[g] = s_l[g] * alpha + sum;
            s_m[g] = mx;
            s_alpha[g] = alpha;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < GMAX / 2; ++k) {
            const int g = g0 + 2 * k;
            if (g < G) {
                float sacc = 0.0f;
                for (int t = 0; t < TILE; ++t) sacc = fmaf(s_p[g][t], s_v[t][d], sacc);
                acc[k] = acc[k] * s_alpha[g] + sacc;
            }
        }
        __syncthreads();
    }

    const Partials pt = partials(a.ws, a.H * G * a.P);
#pragma unroll
    for (int k = 0; k < GMAX / 2; ++k) {
        const int g = g0 + 2 * k;
        if (g < G) pt.o[((int64_t)(h * G + g) * a.P + p) * D + d] = acc[k];
    }
    if (tid < G) pt.ml[(int64_t)(h * G + tid) * a.P + p] = f32x2{s_m[tid], s_l[tid]};
}

// Log-sum-exp merge of the partition partials (_reduce_partials, triton_attention.py:168-181).
// 1-D grid of 64 * ceil(Hq / 8) single-wave workgroups: each merges 16 output
// channels of one query head, the eight channel slices of a head on one XCD.
// Lane (column c4 = lane % 4, partition lane part = lane / 4) owns channels
// 4 c4 .. 4 c4 + 3 and every 16th partition from `part`; a partition costs
// it one 16-byte load of its four channels (the partials' 128-float output
// rows) and one 8-byte load of (m, l) (the pair array after them), nine
// partitions per round, all issued before any arithmetic.  The 16 running
// states of a column then merge inside the wave (two DPP row rotations, two
// permlane swaps): no LDS, no barrier (a four-wave form with an LDS exchange
// measured 0.1 us per layer slower).
constexpr int RED_THREADS = 64;
constexpr int RED_C4 = 4;                          // four-channel columns per workgroup
constexpr int RED_PARTS = RED_THREADS / RED_C4;    // partition lanes
constexpr int RED_BATCH = 9;                       // partitions per lane per round (144 partitions)

__global__ __launch_bounds__(RED_THREADS) void decode_reduce(const float *ws, int64_t P, int Hq, void *out, int odt)
{
    int item, slice;
    iq_xcd_item_slice((int)blockIdx.x, item, slice);    // the 8 channel slices of a head on one XCD
    if (item >= Hq) return;
    const int64_t hq = item;
    const int lane = threadIdx.x, c4 = lane % RED_C4, part = lane / RED_C4;
    const int c0 = slice * (4 * RED_C4) + 4 * c4;
    const Partials pt = partials(const_cast<float *>(ws), (int64_t)Hq * P);
    const float *base = pt.o + hq * P * D;
    const f32x2 *mlb = pt.ml + hq * P;
    const float ninf = -__uint_as_float(0x7f800000u);
    float m = ninf, den = 0.0f;
    f32x4 num = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int p0 = part; p0 < (int)P; p0 += RED_PARTS * RED_BATCH) {
        f32x4 a[RED_BATCH];
        f32x2 ml[RED_BATCH];
#pragma unroll
        for (int k = 0; k < RED_BATCH; ++k) {
            const int pp = min(p0 + RED_PARTS * k, (int)P - 1);
            a[k] = *(const f32x4 *)(base + (int64_t)pp * D + c0);
            ml[k] = mlb[pp];
        }
        float mm = m;
#pragma unroll
        for (int k = 0; k < RED_BATCH; ++k) {
            if (p0 + RED_PARTS * k >= (int)P) ml[k] = f32x2{ninf, 0.0f};
            mm = fmaxf(mm, ml[k].x);
        }
        if (mm == ninf) continue;
        const float wo = m == ninf ? 0.0f : __expf(m - mm);
        num *= wo;
        den *= wo;
#pragma unroll
        for (int k = 0; k < RED_BATCH; ++k) {
            const float w = ml[k].x == ninf ? 0.0f : __expf(ml[k].x - mm);
            num += a[k] * w;
            den = fmaf(ml[k].y, w, den);
        }
        m = mm;
    }
    // lanes with equal lane % 4 hold the 16 partition lanes of one column:
    // rotate by 4 and 8 within each 16-lane row (DPP), then across the rows
    static_assert(RED_C4 == 4 && RED_THREADS == 64, "the DPP rotations assume four columns in one wave");
    float mw = fmaxf(m, dpp_f<0x124>(m));          // row_ror:4
    mw = fmaxf(mw, dpp_f<0x128>(mw));              // row_ror:8
    mw = xmax16(mw);
    const float wt = m == ninf ? 0.0f : __expf(m - mw);
    num *= wt;
    den *= wt;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        num[e] += dpp_f<0x124>(num[e]);
        num[e] = xsum16(num[e] + dpp_f<0x128>(num[e]));
    }
    den += dpp_f<0x124>(den);
    den = xsum16(den + dpp_f<0x128>(den));
    if (lane < RED_C4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) iq_store_as(out, hq * D + c0 + e, num[e] / den, odt);
    }
}

}  // namespace

int iq_decode_fast_launch(const void *q, int q_dtype, int64_t q_stride_h, int64_t Hq, const int64_t *tables,
                          const int8_t *key_map, const int8_t *value_map, int64_t n_blocks, int64_t block_tokens,
                          int64_t H, int64_t S,
                          int value_bits, int value_group, const void *sink_k, const void *sink_v, int64_t sink_k_sh,
                          int64_t sink_k_st, int64_t sink_v_sh, int64_t sink_v_st, int64_t sink_t,
                          const void *tail_k, const void *tail_v, int64_t tail_k_sh, int64_t tail_k_st,
                          int64_t tail_v_sh, int64_t tail_v_st, int64_t tail_t, float scale, float *workspace,
                          void *out, int out_dtype, const iq_block_run *run, int64_t *parts, hipStream_t stream);

namespace {

int64_t partitions(int64_t n_blocks, int64_t sink_t, int64_t tail_t)
{
    return n_blocks + (sink_t + DENSE_SPLIT - 1) / DENSE_SPLIT + (tail_t + DENSE_SPLIT - 1) / DENSE_SPLIT;
}

}  // namespace

extern "C" int64_t iq_decode_workspace_floats(int64_t Hq, int64_t n_blocks, int64_t sink_t, int64_t tail_t)
{
    return Hq * partitions(n_blocks, sink_t, tail_t) * (D + 2);
}


extern "C" int iq_decode_attention(const void *q, int q_dtype, int64_t q_stride_h, int64_t Hq,
                                   const int64_t *tables, const int8_t *key_map, const int8_t *value_map,
                                   const iq_block_run *run, int64_t n_blocks, int64_t block_tokens, int64_t H, int64_t S, int value_bits,
                                   int value_group, const void *sink_k, const void *sink_v, int64_t sink_k_sh,
                                   int64_t sink_k_st, int64_t sink_v_sh, int64_t sink_v_st, int64_t sink_t,
                                   const void *tail_k, const void *tail_v, int64_t tail_k_sh, int64_t tail_k_st,
                                   int64_t tail_v_sh, int64_t tail_v_st, int64_t tail_t, float scale,
                                   float *workspace, int64_t workspace_floats, void *out, int out_dtype,
                                   void *stream)
{
    IQ_CHECK_ARG(q && out && workspace, "iq_decode_attention: null pointer");
    IQ_CHECK_ARG(q_dtype >= IQ_F32 && q_dtype <= IQ_F16, "iq_decode_attention: bad query dtype");
    IQ_CHECK_ARG(out_dtype >= IQ_F32 && out_dtype <= IQ_F16, "iq_decode_attention: bad output dtype");
    IQ_CHECK_ARG(H >= 1 && Hq >= 1 && Hq % H == 0, "iq_decode_attention: Hq %% H != 0");
    const int64_t G = Hq / H;
    IQ_CHECK_ARG(G <= GMAX, "iq_decode_attention: %lld query heads per KV head exceeds %d", (long long)G, GMAX);
    IQ_CHECK_ARG(n_blocks >= 0 && sink_t >= 0 && tail_t >= 0, "iq_decode_attention: negative length");
    IQ_CHECK_ARG(n_blocks == 0 || (tables && key_map && block_tokens >= 1), "iq_decode_attention: no tables");
    IQ_CHECK_ARG(S >= 0 && S <= 64, "iq_decode_attention: S out of range");
    IQ_CHECK_ARG(value_bits == 0 || value_bits == 2 || value_bits == 4, "iq_decode_attention: value_bits");
    IQ_CHECK_ARG(value_bits == 0 || value_group == 32 || value_group == 64 || value_group == 128,
                 "iq_decode_attention: value_group");
    IQ_CHECK_ARG(value_bits != 0 || n_blocks == 0 || value_map, "iq_decode_attention: K4 values need a map");
    IQ_CHECK_ARG(sink_t == 0 || (sink_k && sink_v), "iq_decode_attention: null sink");
    IQ_CHECK_ARG(tail_t == 0 || (tail_k && tail_v), "iq_decode_attention: null tail");
    const int64_t P = partitions(n_blocks, sink_t, tail_t);
    IQ_CHECK_ARG(P >= 1, "iq_decode_attention: attention requires at least one key/value token");
    IQ_CHECK_ARG(P <= 65535, "iq_decode_attention: too many partitions");
    IQ_CHECK_ARG(workspace_floats >= Hq * P * (D + 2), "iq_decode_attention: workspace too small");
    // Matrix-core path for bf16/f16 queries (at most 16 salient channels, 16
    // query heads per KV head); the general kernel covers the rest.
    int64_t parts = P;
    const int fast = iq_decode_fast_launch(q, q_dtype, q_stride_h, Hq, tables, key_map, value_map, n_blocks,
                                           block_tokens, H,
                                           S, value_bits, value_group, sink_k, sink_v, sink_k_sh, sink_k_st,
                                           sink_v_sh, sink_v_st, sink_t, tail_k, tail_v, tail_k_sh, tail_k_st,
                                           tail_v_sh, tail_v_st, tail_t, scale, workspace, out, out_dtype, run,
                                           &parts, (hipStream_t)stream);
    if (fast == IQ_OK) {
        IQ_CHECK_LAUNCH("decode_fast");
        if (parts == 1) return IQ_OK;
    } else {
        DecodeArgs a{q, q_dtype, q_stride_h, Hq, tables, key_map, value_map, n_blocks, block_tokens, H, S,
                     value_bits, value_group, sink_k, sink_v, sink_k_sh, sink_k_st, sink_v_sh, sink_v_st, sink_t,
                     tail_k, tail_v, tail_k_sh, tail_k_st, tail_v_sh, tail_v_st, tail_t, scale, workspace, P,
                     (int)G, out, out_dtype};
        hipLaunchKernelGGL(decode_partials_generic, dim3((unsigned)H, (unsigned)P), dim3(DA_THREADS), 0,
                           (hipStream_t)stream, a);
        IQ_CHECK_LAUNCH("decode_partials_generic");
    }
    static_assert(D / (4 * RED_C4) == 8, "eight channel slices per head");
    hipLaunchKernelGGL(decode_reduce, dim3((unsigned)(64 * ((Hq + 7) / 8))), dim3(RED_THREADS), 0,
                       (hipStream_t)stream, workspace, parts, (int)Hq, out, out_dtype);
    IQ_CHECK_LAUNCH("decode_reduce");
    return IQ_OK;
}

extern "C" int iq_decode_merge(const float *workspace, int64_t parts, int64_t Hq, void *out, int out_dtype,
                               void *stream)
{
    IQ_CHECK_ARG(workspace && out, "iq_decode_merge: null pointer");
    IQ_CHECK_ARG(parts >= 1 && parts <= 65535 && Hq >= 1, "iq_decode_merge: bad sizes");
    IQ_CHECK_ARG(out_dtype >= IQ_F32 && out_dtype <= IQ_F16, "iq_decode_merge: bad output dtype");
    hipLaunchKernelGGL(decode_reduce, dim3((unsigned)(64 * ((Hq + 7) / 8))), dim3(RED_THREADS), 0,
                       (hipStream_t)stream, workspace, parts, (int)Hq, out, out_dtype);
    IQ_CHECK_LAUNCH("decode_reduce");
    return IQ_OK;
}

extern "C" int64_t iq_decode_partitions(int64_t n_blocks, int64_t sink_t, int64_t tail_t, int fast)
{
    return fast ? n_blocks + (sink_t + tail_t + DENSE_SPLIT - 1) / DENSE_SPLIT : partitions(n_blocks, sink_t, tail_t);
}

// ---------------------------------------------------------------- allocation-free variant
//
// Scratch of iq_decode_attention_noalloc: the partition partials live in this
// file-scope device array instead of a caller workspace.  Each GPU the library
// runs on holds its own copy (IQ_NOALLOC_SCRATCH_FLOATS floats) until the
// process ends.  Host code never passes `scratch` itself to a kernel: its
// per-device address comes from hipGetSymbolAddress, taken once per device
// with that device current.  The partials are fully written by the first
// kernel before the merge kernel reads them, so nothing needs clearing
// between calls; calls that overlap on one GPU share the array and race.
static __device__ __align__(256) float scratch[IQ_NOALLOC_SCRATCH_FLOATS];

namespace {

constexpr int SCRATCH_DEVICES = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[SCRATCH_DEVICES] = {};

// Address of this device's copy of `scratch`, or nullptr after recording an error.
float *device_scratch()
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_DEVICES) {
        iq_fail(IQ_ERR_DEVICE, "iq_decode_attention_noalloc: no current device below %d", SCRATCH_DEVICES);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            iq_fail(IQ_ERR_DEVICE, "iq_decode_attention_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = (float *)p;
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int iq_decode_attention_noalloc(const void *q, int q_dtype, int64_t q_stride_h, int64_t Hq,
                                           const int64_t *tables, const int8_t *key_map, const int8_t *value_map,
                                           const iq_block_run *run, int64_t n_blocks, int64_t block_tokens, int64_t H, int64_t S,
                                           int value_bits, int value_group, const void *sink_k, const void *sink_v,
                                           int64_t sink_k_sh, int64_t sink_k_st, int64_t sink_v_sh,
                                           int64_t sink_v_st, int64_t sink_t, const void *tail_k,
                                           const void *tail_v, int64_t tail_k_sh, int64_t tail_k_st,
                                           int64_t tail_v_sh, int64_t tail_v_st, int64_t tail_t, float scale,
                                           void *out, int out_dtype, void *stream)
{
    IQ_CHECK_ARG(Hq >= 1 && n_blocks >= 0 && sink_t >= 0 && tail_t >= 0, "iq_decode_attention_noalloc: bad sizes");
    const int64_t need = Hq * partitions(n_blocks, sink_t, tail_t) * (D + 2);
    IQ_CHECK_ARG(need <= IQ_NOALLOC_SCRATCH_FLOATS,
                 "iq_decode_attention_noalloc: %lld query heads x %lld partitions need %lld scratch floats; the "
                 "static scratch holds %lld (use iq_decode_attention with a workspace)",
                 (long long)Hq, (long long)partitions(n_blocks, sink_t, tail_t), (long long)need,
                 (long long)IQ_NOALLOC_SCRATCH_FLOATS);
    float *ws = device_scratch();
    if (!ws) return IQ_ERR_DEVICE;
    return iq_decode_attention(q, q_dtype, q_stride_h, Hq, tables, key_map, value_map, run, n_blocks, block_tokens, H, S,
                               value_bits, value_group, sink_k, sink_v, sink_k_sh, sink_k_st, sink_v_sh, sink_v_st,
                               sink_t, tail_k, tail_v, tail_k_sh, tail_k_st, tail_v_sh, tail_v_st, tail_t, scale,
                               ws, IQ_NOALLOC_SCRATCH_FLOATS, out, out_dtype, stream);
}
