// Fused packed-KV decode attention on matrix cores (gfx950, bf16/f16 queries).
//
// Same semantics and partial format as decode_partials_generic
// (triton_attention.py:67-165): one workgroup per (KV head, partition),
// partitions = packed blocks then 32-token slices of sink and tail; keys and
// values are decoded and rounded to the query dtype exactly as the
// dequantize-then-attend path does.  Each of the 4 wavefronts owns a
// 64-token chunk of the partition.
//
//   * Every global load of a workgroup (pointer-table row, then payload,
//     scales, roles, descriptors, query rows) is issued up front; one
//     barrier publishes the block metadata in LDS before any arithmetic.
//   * K payload rows arrive as 16-byte loads: lane (t = l%16, q = l/16) holds
//     channels 32q..32q+31 of token t, which is exactly the A operand of four
//     v_mfma_f32_16x16x32 (rows = tokens, k = channels, B = Q^T).
//   * Normal channels decode with one fma per element: the fp8 converter maps
//     a nibble byte n to n * 2^-9 exactly, so fma(v, s * 2^9, -8 s) is the
//     single rounding of (n - 8) * s, as the reference's fp32 multiply.
//   * Salient and donor channels decode to zero in the 4-bit pass (zero
//     constants).  Their 8-bit codes come from the matrix cores: an int8
//     v_mfma_i32_16x16x64 of a selection matrix (16 at a source's channel,
//     1 at its donor's) with the raw nibble bytes gives 16 hi + lo exactly,
//     already in the A-operand layout of the v_mfma_f32_16x16x16 that adds
//     the salient terms; a per-block constant adds q . round(padding) for
//     donors.
//   * Blocks of one batched encode sit at a fixed stride from each other;
//     for that leading run of blocks the addresses come from the kernel
//     arguments, so the payload loads do not wait for a pointer-table row.
//   * LDS stays within 40 KiB (the query rows live in a V tile until every
//     lane holds its operands), so four workgroups share a compute unit.
//   * Online softmax in the log2 domain; P = hi + lo (two bf16/f16 terms) so
//     the P.V product keeps ~16 significant bits of the weights.
//   * Values decode with the same fp8 trick into a 16-row LDS tile per half
//     chunk (row q pairs tokens q and q + 16, rows 132 dwords apart: 16-byte
//     stores and 32-lane reads are free of bank conflicts), read back
//     transposed as the A operand of O^T = V^T P^T.  Group-wise values
//     (V2/V4) take a per-token scale and offset; K4-coded values (the codec
//     of the keys) take per-channel constants, their salient channels come
//     from the int8 selection product with the payload as A operand (which
//     leaves the codes in the k-slot layout of P^T, no LDS), and a donor
//     channel's column is round(pad) * sum(p).
#include "decode_common.h"

#include <atomic>

namespace {

constexpr int D = 128;
constexpr int WAVES = 4;
constexpr int CHUNK = 64;              // tokens per wavefront per pass
constexpr int VR = 132;                // dwords per staged token-pair row of decoded V (128 + 4: rows 4 banks apart)
constexpr int SELROW = D + 16;         // bytes per selection-matrix row (+16: the 16 rows of a read hit distinct banks)
constexpr int OROW = 132;              // floats per staged output row in the combine (128 + 4: conflict-free 16-byte stores)
constexpr int KC_STRIDE = 68;          // float2 slots per 32-channel group of K constants (+4: no bank overlap)
// Dense (sink ++ tail) partitions are 32 tokens: they are dispatched after
// the packed blocks, into the slots left once every packed workgroup is
// resident (or beside two packed workgroups on a compute unit), so a short
// one adds the least time after the packed workgroups finish.
constexpr int DENSE_SPLIT = 32;
constexpr int QROW = D + 8;            // u16 per staged query row (+8: the 16 rows of a B-operand read hit distinct banks)
constexpr float LN2 = 0.693147180559945309f;


struct FastArgs {
    // the leading run of blocks laid out at a fixed stride (a batched encode):
    // block p < run_blocks has field f (pointer-table column order) at
    // run[f] + p * (that field's bytes per block)
    const uint8_t *run[IQ_TABLE_COLS];
    int64_t run_blocks;
    const uint16_t *q;
    int64_t q_sh;
    int G;
    const int64_t *tables;
    const int8_t *kmap, *vmap;   // role maps of keys and (K4-coded) values
    int64_t nblk, BT, H, S;
    int vshift;      // log2 of the value group (32, 64 or 128 channels)
    const uint16_t *sk, *sv;
    int64_t sk_sh, sk_st, sv_sh, sv_st, sink_t;
    const uint16_t *tk, *tv;
    int64_t tk_sh, tk_st, tv_sh, tv_st, tail_t;
    float c_log2;    // softmax scale * log2(e)
    float *ws;
    int64_t P;
    void *out;       // final [Hq, 128] output when there is one partition
    int odt;
    // 1 when the grid holds more workgroups than fit on the device at once:
    // the dense partitions then take the first grid rows and keep the top
    // issue priority, so they finish early and the packed workgroups left
    // over start early instead of after the resident ones
    int dense_first;
};

// Partition of grid row y: packed blocks, then dense slices; or, with
// dense_first, the dense slices first.
__device__ __forceinline__ int64_t partition_of(const FastArgs &a, int64_t y)
{
    const int64_t nd = a.P - a.nblk;
    return a.dense_first ? (y < nd ? a.nblk + y : y - nd) : y;
}

// Workgroup LDS, shared by the packed and the dense instantiation of the body.
// At most 40 KiB, so that four workgroups share a compute unit.
struct __attribute__((aligned(16))) FastSmem {
    // per wavefront: staged decoded V as [token pair][channel] dwords (two
    // tokens of one channel per dword: pair row q of half chunk m holds
    // tokens 32 m + q and 32 m + 16 + q); also the final combine.  Until
    // every lane holds its operands, wave 0's tile holds the query rows
    // (dtype bits, QROW halves per row, zero beyond G) and waves 1 and 2's
    // tiles the selection matrices of the key and the value salient codes.
    uint32_t v[WAVES][16 * VR];
    f32x2 kc[4 * KC_STRIDE];     // per channel (s * 2^9, -8 s); (0, 0) at salient and donor channels
    int8_t role[D];
    uint32_t salw[16];           // source k: its channel | donor channel << 8
    f32x2 salf[16];              // (s_src, -128 s_src)
    uint16_t qsal[16 * 20];      // Q[g][src_k], zero beyond S
    float dpad[16];              // padding of donor k, rounded to the query dtype
    float bias[16];              // per query row: sum_k q[g][donor k] * dpad[k]
    // K4-coded values: per-channel constants as for keys, the value role map,
    // and per descriptor k the source's (s, -128 s), the donor's rounded
    // padding and both channels
    f32x2 vc[4 * KC_STRIDE];
    int8_t vrole[D];
    f32x2 vsalf[16];
    float vdpad[16];
    int vsrc[16], vdon[16];
    float wm[WAVES][16], wl[WAVES][16];
};
static_assert(sizeof(FastSmem) <= 40 * 1024, "four workgroups per compute unit");
static_assert(16 * QROW / 2 <= 16 * VR, "the query rows fit in one wave's tile");
static_assert(16 * SELROW <= 16 * VR * 4, "the salient selection matrix fits in one wave's tile");
static_assert(16 * OROW <= 16 * VR, "the combine's output rows fit in one wave's tile");


// One partition.  PACKED and dense partitions are separate instantiations so
// that neither has a branch between its loads and their first use: a branch
// join there makes the compiler wait for every load in flight.
//
// VBITS 2 or 4: group-wise values (value_codec.py); VBITS 0: K4-coded values
// (codec.py), decoded like the keys (triton_attention.py:33-51).
template <bool F16, int VBITS, bool PACKED>
__device__ __forceinline__ void fast_body(const FastArgs &a, FastSmem &sm)
{
    constexpr bool K4V = VBITS == 0;
    constexpr int VROW = K4V ? D / 2 : D * VBITS / 8;   // V payload bytes per token
    constexpr int VQ = VROW / 4;                 // bytes per 32-channel quarter row
    constexpr int VQW = VQ / 4;                  // dwords per quarter row

    uint32_t (&s_v)[WAVES][16 * VR] = sm.v;
    uint16_t *const s_q = (uint16_t *)&sm.v[0][0];
    f32x2 *const s_kc = sm.kc;
    int8_t *const s_role = sm.role;
    uint32_t *const s_salw = sm.salw;
    f32x2 *const s_salf = sm.salf;
    uint16_t *const s_qsal = sm.qsal;
    float *const s_dpad = sm.dpad;
    float *const s_bias = sm.bias;
    f32x2 *const s_vc = sm.vc;
    float (&s_wm)[WAVES][16] = sm.wm;
    float (&s_wl)[WAVES][16] = sm.wl;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Issue priority falls as a wavefront advances through its phases, so
    // the workgroups sharing a compute unit progress together instead of the
    // oldest finishing first and leaving the last one alone to run latency-bound.
    __builtin_amdgcn_s_setprio(3);
    const int gl = lane & 15, ql = lane >> 4;     // MFMA column (query row / channel) and k-slot group
    // V writer of group-wise values and dense rows: pair row pl (tokens
    // 32 m + pl and 32 m + 16 + pl) and 32-channel quarter qq
    const int pl = lane & 15, qq = lane >> 4;
    const int h = blockIdx.x;
    const int64_t p = partition_of(a, blockIdx.y);
    const int G = a.G;
    // the fp8 converter maps byte n < 16 to n * 2^-9 exactly (e4m3 subnormals
    // and the first binade), so scales are pre-multiplied by 2^9
    constexpr float inv_unit = 512.0f;
    const int ngroups = D >> a.vshift;

    // ---------------- geometry (wave-uniform) and every global load up front
    // All loads are unconditional (indices clamped into range) and issued
    // before any of them is consumed: the query row, then the block's
    // per-channel constants, then the payload, so one round trip after the
    // pointer-table row covers all of them.  Rows past the end of a partition
    // load a clamped valid row; their logits are masked to -inf, so they get
    // weight exactly 0.
    constexpr bool packed = PACKED;
    const uint8_t *kpay = nullptr, *vpay = nullptr;
    const uint16_t *vsc = nullptr, *voff = nullptr;
    int start = 0, stop = 0;
    const int S = packed ? (int)a.S : 0;         // at most 16 (one group of salient channels)
    const int qg = tid >> 4, qc = (tid & 15) * 8;  // this thread's 8 query elements
    const u32x4 qraw = ld16(a.q + (int64_t)(h * G + (qg < G ? qg : G - 1)) * a.q_sh + qc);
    float kscale = 0.0f, kpad = 0.0f, vscale = 0.0f, vpad = 0.0f;
    uint32_t krole = 0u, ksrc = 0u, kdon = 0u, vrole = 0u;
    int base = 0;
    u32x4 kw[4];
    u32x4 vk[4];                                   // K4-coded values: laid out as kw
    uint32_t vw[2][2][VQW];                        // [half chunk][token of the pair][dword]
    uint32_t vp[2][2][2];                          // [half chunk][token of the pair][scale, offset] (f16 bits)
#define IQ_LOAD_CHUNK(b_)                                                                             \
    do {                                                                                              \
        const int b0 = (b_);                                                                          \
        _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                               \
            const int t = min(b0 + 16 * j + gl, stop - 1);                                            \
            kw[j] = ldnt_at<u32x4>(kpay, (uint32_t)(t * (D / 2) + 16 * ql));                          \
            if constexpr (K4V) vk[j] = ldnt_at<u32x4>(vpay, (uint32_t)(t * (D / 2) + 16 * ql));       \
        }                                                                                             \
        const int gi = (32 * qq) >> a.vshift;                                                         \
        _Pragma("unroll") for (int m = 0; m < (K4V ? 0 : 2); ++m) {                                   \
            _Pragma("unroll") for (int u = 0; u < 2; ++u) {                                           \
                const int t = min(b0 + 32 * m + 16 * u + pl, stop - 1);                               \
                const uint32_t vo = (uint32_t)(t * VROW + VQ * qq);                                   \
                if constexpr (VQW == 2) {                                                             \
                    const u32x2 r = ldnt_at<u32x2>(vpay, vo);                                         \
                    vw[m][u][0] = r[0];                                                               \
                    vw[m][u][1] = r[1];                                                               \
                } else {                                                                              \
                    const u32x4 r = ldnt_at<u32x4>(vpay, vo);                                         \
                    _Pragma("unroll") for (int w = 0; w < VQW; ++w) vw[m][u][w] = r[w];               \
                }                                                                                     \
                vp[m][u][0] = ldg_at<uint16_t>(vsc, (uint32_t)(2 * (t * ngroups + gi)));              \
                vp[m][u][1] = ldg_at<uint16_t>(voff, (uint32_t)(2 * (t * ngroups + gi)));             \
            }                                                                                         \
        }                                                                                             \
    } while (0)
    if (packed) {
        // block addresses: from the kernel arguments for the run of
        // fixed-stride blocks, else one 64-byte scalar load of the pointer-table
        // row (written by an earlier launch, so the kernel-start cache
        // invalidation covers it)
        uintptr_t tr[IQ_TABLE_COLS];
        if (p < a.run_blocks) {
            // bytes per block of each field: K payload, K scales, K padding,
            // V payload, V scales, V offsets (K4 values: V padding), K sources, K donors
            const int64_t HB = a.H * a.BT;
            const int64_t per[IQ_TABLE_COLS] = {HB * (D / 2), a.H * D * 4, a.H * a.S * 4, HB * VROW,
                                                K4V ? a.H * D * 4 : HB * ngroups * 2,
                                                K4V ? a.H * a.S * 4 : HB * ngroups * 2, a.H * a.S, a.H * a.S};
#pragma unroll
            for (int k = 0; k < IQ_TABLE_COLS; ++k) tr[k] = (uintptr_t)(a.run[k] + p * per[k]);
        } else {
            const __attribute__((address_space(4))) int64_t *rv =
                (const __attribute__((address_space(4))) int64_t *)(a.tables + p * IQ_TABLE_COLS);
#pragma unroll
            for (int k = 0; k < IQ_TABLE_COLS; ++k) tr[k] = (uintptr_t)rv[k];
        }
        auto row = [&](int k) -> uintptr_t { return tr[k]; };
        krole = (uint8_t)ldg<int8_t>(a.kmap + (p * a.H + h) * D + (tid & (D - 1)));
        kscale = ldg<float>((const float *)row(1) + h * D + (tid & (D - 1)));
        {   // no branch around these loads: with S == 0 they read valid
            // addresses (the role map, the scales) whose values go unused
            const int k = tid < S ? tid : (S > 0 ? S - 1 : 0);
            const uint8_t *srcs = S > 0 ? (const uint8_t *)row(6) + h * S : (const uint8_t *)a.kmap;
            const uint8_t *dons = S > 0 ? (const uint8_t *)row(7) + h * S : (const uint8_t *)a.kmap;
            const float *pads = S > 0 ? (const float *)row(2) + h * S : (const float *)row(1);
            ksrc = ldg<uint8_t>(srcs + k);
            kdon = ldg<uint8_t>(dons + k);
            kpad = ldg<float>(pads + k);
            if constexpr (K4V) {
                vrole = (uint8_t)ldg<int8_t>(a.vmap + (p * a.H + h) * D + (tid & (D - 1)));
                vscale = ldg<float>((const float *)row(4) + h * D + (tid & (D - 1)));
                vpad = ldg<float>(S > 0 ? (const float *)row(5) + h * S + k : (const float *)row(4));
            }
        }
        kpay = (const uint8_t *)row(0) + (int64_t)h * a.BT * (D / 2);
        vpay = (const uint8_t *)row(3) + (int64_t)h * a.BT * VROW;
        vsc = (const uint16_t *)row(4) + (int64_t)h * a.BT * ngroups;
        voff = (const uint16_t *)row(5) + (int64_t)h * a.BT * ngroups;
        stop = (int)a.BT;
        base = CHUNK * wave;
        IQ_LOAD_CHUNK(base);                        // clamped: also for waves past the end
        // keep every use of the small loads below the payload issue
        asm volatile("" ::: "memory");
    } else {
        // dense partitions cover sink ++ tail as one token sequence
        const int length = (int)(a.sink_t + a.tail_t);
        start = (int)((p - a.nblk) * DENSE_SPLIT);
        stop = start + DENSE_SPLIT < length ? start + DENSE_SPLIT : length;
        base = start + CHUNK * wave;
    }
    // row t (already clamped into [0, stop)) of the dense key / value sequence
    const int nsink = (int)a.sink_t;
    auto dense_k = [&](int t) {
        return t < nsink ? a.sk + h * a.sk_sh + (int64_t)t * a.sk_st : a.tk + h * a.tk_sh + (int64_t)(t - nsink) * a.tk_st;
    };
    auto dense_v = [&](int t) {
        return t < nsink ? a.sv + h * a.sv_sh + (int64_t)t * a.sv_st : a.tv + h * a.tv_sh + (int64_t)(t - nsink) * a.tv_st;
    };
    // consume the small loads (the payload stays in flight)
    *(u32x4 *)(s_q + qg * QROW + qc) = qg < G ? qraw : u32x4{0u, 0u, 0u, 0u};
    // selection matrix of the salient codes, [source k][channel] bytes with the
    // even channels of a row first (channel c at byte (c & 1) * 64 + c / 2),
    // staged in wave 1's V tile, which is free until the operands are loaded
    uint8_t *const s_sel = (uint8_t *)&sm.v[1][0];
    uint8_t *const s_vsel = (uint8_t *)&sm.v[2][0];  // the same for K4-coded values
    if (packed && tid < 16 * SELROW / 16) *(u32x4 *)(s_sel + 16 * tid) = u32x4{0u, 0u, 0u, 0u};
    if (packed && K4V && tid < 16 * SELROW / 16) *(u32x4 *)(s_vsel + 16 * tid) = u32x4{0u, 0u, 0u, 0u};
    if (packed) {
        if (tid < D) {
            // salient and donor channels decode to zero in the 4-bit pass:
            // their terms come from the 8-bit codes and the donor padding
            s_kc[(tid >> 5) * KC_STRIDE + (tid & 31)] =
                krole == 0xffu ? f32x2{kscale * inv_unit, -8.0f * kscale} : f32x2{0.0f, 0.0f};
            s_role[tid] = (int8_t)krole;
        }
        if (tid < S) {
            s_salw[tid] = ksrc | (kdon << 8);
            s_dpad[tid] = round_q<F16>(kpad);
        }
        if constexpr (K4V) {
            if (tid < D) {
                s_vc[(tid >> 5) * KC_STRIDE + (tid & 31)] =
                    vrole == 0xffu ? f32x2{vscale * inv_unit, -8.0f * vscale} : f32x2{0.0f, 0.0f};
                sm.vrole[tid] = (int8_t)vrole;
            }
            if (tid < S) sm.vdpad[tid] = round_q<F16>(vpad);
        }
    }
    __syncthreads();

    // ---------------- cooperative per-workgroup constants
    if constexpr (PACKED) {
        // a source channel's descriptor index is -2 - role[its donor]; a
        // donor's is -2 - its role.  Each marks its byte of the selection
        // matrix: 16 for the source (high nibble), 1 for the donor.
        if (tid < D) {
            const int r = (int)(int8_t)krole;
            const int k = r >= 0 ? -2 - (int)s_role[r] : -2 - r;
            if (k >= 0 && k < S) {
                s_sel[k * SELROW + (tid & 1) * (D / 2) + (tid >> 1)] = r >= 0 ? 16 : 1;
                if (r >= 0) s_salf[k] = f32x2{kscale, -128.0f * kscale};   // exact
            }
        }
        {   // thread (query row g, descriptor k): the source's query value, and
            // the donor term q[g][donor k] * round(pad k) summed over the row's 16 lanes
            const int g = tid >> 4, k = tid & 15;
            const bool live = k < S;
            const uint32_t sw = live ? s_salw[k] : 0u;
            s_qsal[g * 20 + k] = live ? s_q[g * QROW + (sw & 0xffu)] : (uint16_t)0;
            const float t = row_sum16(live ? to_f32<F16>(s_q[g * QROW + (sw >> 8)]) * s_dpad[k] : 0.0f);
            if (k == 0) s_bias[g] = t;
        }
        if (tid >= S && tid < 16) s_salf[tid] = f32x2{0.0f, 0.0f};
        if constexpr (K4V) {
            // the value role map marks the value selection matrix the same way;
            // each descriptor also records its source and donor channel
            if (tid < D) {
                const int r = (int)(int8_t)vrole;
                const int k = r >= 0 ? -2 - (int)sm.vrole[r] : -2 - r;
                if (k >= 0 && k < S) {
                    s_vsel[k * SELROW + (tid & 1) * (D / 2) + (tid >> 1)] = r >= 0 ? 16 : 1;
                    if (r >= 0) {
                        sm.vsalf[k] = f32x2{vscale, -128.0f * vscale};
                        sm.vsrc[k] = tid;
                    } else {
                        sm.vdon[k] = tid;
                    }
                }
            }
            if (tid >= S && tid < 16) sm.vsalf[tid] = f32x2{0.0f, 0.0f};
        }
    }
    __syncthreads();

    // ---------------- per-lane constants
    u32x4 qb[4];                                   // B operand: Q[g = gl][32 ql + 8 d + e]
#pragma unroll
    for (int d = 0; d < 4; ++d) qb[d] = *(const u32x4 *)(s_q + gl * QROW + 32 * ql + 8 * d);
    const float bias = PACKED ? s_bias[gl] : 0.0f;  // sum_k q[gl][don_k] * round(pad_k)
    // salient operands: the selection matrix rows (source k = gl; byte i of
    // sel_e / sel_o is channel 32 ql + 2 i / 32 ql + 2 i + 1: 16 at the
    // source's channel, 1 at its donor's), the query values of the sources
    // (B operand, k = 4 ql + e) and the codes' (scale, -128 scale)
    i32x4 sel_e = {0, 0, 0, 0}, sel_o = {0, 0, 0, 0};
    u32x2 qs = {0u, 0u};
    f32x2 sf[4];
    if (PACKED && S > 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) sf[e] = s_salf[4 * ql + e];
        qs = *(const u32x2 *)(s_qsal + gl * 20 + 4 * ql);
        sel_e = *(const i32x4 *)(s_sel + gl * SELROW + 16 * ql);
        sel_o = *(const i32x4 *)(s_sel + gl * SELROW + D / 2 + 16 * ql);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) sf[e] = f32x2{0.0f, 0.0f};
    }
    // K4-coded values: the value selection rows (as B operand: source gl) and
    // the (s, -128 s) of source gl
    i32x4 vsel_e = {0, 0, 0, 0}, vsel_o = {0, 0, 0, 0};
    f32x2 vsf = {0.0f, 0.0f};
    if (PACKED && K4V && S > 0) {
        vsel_e = *(const i32x4 *)(s_vsel + gl * SELROW + 16 * ql);
        vsel_o = *(const i32x4 *)(s_vsel + gl * SELROW + D / 2 + 16 * ql);
        vsf = sm.vsalf[gl];
    }
    // every lane holds its operands: the tiles of waves 0-2 may now be overwritten
    __syncthreads();

    float m_run = NEG_INF, l_run = 0.0f;
    f32x4 acc[8];                                  // O^T rows 16 n + 4 ql + r, column gl (unscaled)
    f32x4 acc_sal = {0.0f, 0.0f, 0.0f, 0.0f};      // K4 values: O^T rows = sources 4 ql + r, column gl

    uint32_t *vt = s_v[wave];
    // The P.V operand reads: volatile, so that each lane's four pair rows
    // stay four single-dword LDS reads straight into the operand registers
    // (the compiler would otherwise pair the reads of channel tiles n and
    // n + 1 and copy every operand into place).
    const volatile __attribute__((address_space(3))) uint32_t *const vtile =
        (const volatile __attribute__((address_space(3))) uint32_t *)vt;

    // one pass: a partition holds at most CHUNK * WAVES tokens
    if (base < stop) {
        const bool full = base + CHUNK <= stop;
        // ---------------- logits S^T[token, g] for four 16-token tiles
        f32x4 sc[4];
        if (packed) {
            // Per 16-token tile j and 32-channel group d: kv = K rows of the tile,
            // channels 32 ql + 8 d .. + 7, rounded to the query dtype.
            auto k_operand = [&](uint32_t x, const f32x2 *kc) {
                const u32x4 c01 = *(const u32x4 *)(kc + 0), c23 = *(const u32x4 *)(kc + 2);
                const u32x4 c45 = *(const u32x4 *)(kc + 4), c67 = *(const u32x4 *)(kc + 6);
                const uint32_t lo = x & 0x0f0f0f0fu, hi = (x >> 4) & 0x0f0f0f0fu;
                const f32x2 e01 = fp8x2<false>(lo), e23 = fp8x2<true>(lo);
                const f32x2 o01 = fp8x2<false>(hi), o23 = fp8x2<true>(hi);
#define KF(cv, i) __uint_as_float(cv[i])
                u32x4 kv;
                kv[0] = pack2<F16>(fmaf(e01.x, KF(c01, 0), KF(c01, 1)), fmaf(o01.x, KF(c01, 2), KF(c01, 3)));
                kv[1] = pack2<F16>(fmaf(e01.y, KF(c23, 0), KF(c23, 1)), fmaf(o01.y, KF(c23, 2), KF(c23, 3)));
                kv[2] = pack2<F16>(fmaf(e23.x, KF(c45, 0), KF(c45, 1)), fmaf(o23.x, KF(c45, 2), KF(c45, 3)));
                kv[3] = pack2<F16>(fmaf(e23.y, KF(c67, 0), KF(c67, 1)), fmaf(o23.y, KF(c67, 2), KF(c67, 3)));
#undef KF
                return kv;
            };
            // salient terms of tile j: codes 16 hi + lo of sources 4 ql .. 4 ql + 3
            // for token 16 j + gl from the raw nibbles (even / odd channels)
            auto salient = [&](int j, f32x4 acc_j) {
                i32x4 lo4, hi4;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    lo4[d] = (int)(kw[j][d] & 0x0f0f0f0fu);
                    hi4[d] = (int)((kw[j][d] >> 4) & 0x0f0f0f0fu);
                }
                i32x4 code = __builtin_amdgcn_mfma_i32_16x16x64_i8(sel_e, lo4, i32x4{0, 0, 0, 0}, 0, 0, 0);
                code = __builtin_amdgcn_mfma_i32_16x16x64_i8(sel_o, hi4, code, 0, 0, 0);
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = fmaf((float)code[e], sf[e].x, sf[e].y);
                return mma16<F16>(u32x2{pack2<F16>(v[0], v[1]), pack2<F16>(v[2], v[3])}, qs, acc_j);
            };
            // Per tile the sum keeps one order: bias, groups 0..3, salient terms.
#pragma unroll
            for (int j = 0; j < 4; ++j) sc[j] = f32x4{bias, bias, bias, bias};
            if constexpr (VBITS == 2) {
                // group outer: the 8 constants of group d (four distinct LDS
                // addresses per read: broadcasts) are read once and serve the
                // four tiles, whose accumulations are independent matrix-core chains
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    // keeps this group's constant reads here: hoisted, all 64 would stay live
                    asm volatile("" ::: "memory");
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        sc[j] = mma32<F16>(k_operand(kw[j][d], s_kc + ql * KC_STRIDE + 8 * d), qb[d], sc[j]);
                }
                if (S > 0) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) sc[j] = salient(j, sc[j]);
                }
            } else {
                // 4-bit values hold twice the V payload in registers: tile outer
                // keeps one tile's constants live at a time (re-read per tile)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        asm volatile("" ::: "memory");
                        sc[j] = mma32<F16>(k_operand(kw[j][d], s_kc + ql * KC_STRIDE + 8 * d), qb[d], sc[j]);
                    }
                    if (S > 0) sc[j] = salient(j, sc[j]);
                }
            }
        } else {
            // dense sink / tail: K rows of the query dtype are the A operand
            // directly; two tiles' rows (clamped in range, zeroed past the
            // end) are in flight together
#pragma unroll
            for (int j2 = 0; j2 < 4; j2 += 2) {
                u32x4 kd[2][4];
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const int t = base + 16 * (j2 + jj) + gl;
                    const int tc = t < stop ? t : stop - 1;
#pragma unroll
                    for (int d = 0; d < 4; ++d) kd[jj][d] = ld16(dense_k(tc) + 32 * ql + 8 * d);
                }
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const bool ok = base + 16 * (j2 + jj) + gl < stop;
                    f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int d = 0; d < 4; ++d) s = mma32<F16>(ok ? kd[jj][d] : u32x4{0u, 0u, 0u, 0u}, qb[d], s);
                    sc[j2 + jj] = s;
                }
            }
        }

        if (PACKED || !a.dense_first) __builtin_amdgcn_s_setprio(2);
        // ---------------- online softmax (log2 domain); lane holds g = gl, tokens 16 j + 4 ql + r
        // raw logits: the scale is positive, so the maximum commutes with it
        // and is applied once; p = 2^(s c - m) with one fma per logit
        float cmax = NEG_INF;
        if (!full) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (base + 16 * j + 4 * ql + r >= stop) sc[j][r] = NEG_INF;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) cmax = fmaxf(cmax, sc[j][r]);
        const float m_new = xmax16(cmax) * a.c_log2;   // one pass per wavefront: nothing to rescale
        float lsum = 0.0f;
        float pr[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pr[j][r] = __builtin_amdgcn_exp2f(fmaf(sc[j][r], a.c_log2, -m_new));
                lsum += pr[j][r];
            }
        // B operand of half chunk m: k-slot pair r = tokens 32 m + 4 ql + r and
        // 32 m + 16 + 4 ql + r (tiles 2 m and 2 m + 1)
        u32x4 phi[2], plo[2];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t hh = pack2<F16>(pr[2 * m][r], pr[2 * m + 1][r]);
                phi[m][r] = hh;
                plo[m][r] = pack2<F16>(pr[2 * m][r] - to_f32<F16>(hh & 0xffffu),
                                       pr[2 * m + 1][r] - to_f32<F16>(hh >> 16));
            }
        l_run = lsum;
        m_run = m_new;

        // ---------------- two half chunks: decode 32 V rows to LDS, then O^T += V^T P^T
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            uint32_t *dst = vt + pl * VR + 32 * qq;    // pair row pl, channels 32 qq .. 32 qq + 31
            if (m > 0) wave_lds_sync();                // every lane has read half chunk m - 1
            if (packed && K4V) {
                // pair row gl (tokens 16 (2 m) + gl and 16 (2 m + 1) + gl: this
                // lane's rows of tiles 2 m and 2 m + 1), channels 32 ql + 8 d + i,
                // normal channels only (salient and donor channels decode to 0)
                uint32_t *drow = vt + gl * VR + 32 * ql;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    asm volatile("" ::: "memory");
                    const f32x2 *vcp = s_vc + ql * KC_STRIDE + 8 * d;
                    const u32x4 c01 = *(const u32x4 *)(vcp + 0), c23 = *(const u32x4 *)(vcp + 2);
                    const u32x4 c45 = *(const u32x4 *)(vcp + 4), c67 = *(const u32x4 *)(vcp + 6);
                    float val[2][8];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const uint32_t x = vk[2 * m + u][d];
                        const uint32_t lo = x & 0x0f0f0f0fu, hi = (x >> 4) & 0x0f0f0f0fu;
                        const f32x2 e01 = fp8x2<false>(lo), e23 = fp8x2<true>(lo);
                        const f32x2 o01 = fp8x2<false>(hi), o23 = fp8x2<true>(hi);
#define KF(cv, i) __uint_as_float(cv[i])
                        val[u][0] = fmaf(e01.x, KF(c01, 0), KF(c01, 1));
                        val[u][1] = fmaf(o01.x, KF(c01, 2), KF(c01, 3));
                        val[u][2] = fmaf(e01.y, KF(c23, 0), KF(c23, 1));
                        val[u][3] = fmaf(o01.y, KF(c23, 2), KF(c23, 3));
                        val[u][4] = fmaf(e23.x, KF(c45, 0), KF(c45, 1));
                        val[u][5] = fmaf(o23.x, KF(c45, 2), KF(c45, 3));
                        val[u][6] = fmaf(e23.y, KF(c67, 0), KF(c67, 1));
                        val[u][7] = fmaf(o23.y, KF(c67, 2), KF(c67, 3));
#undef KF
                    }
#pragma unroll
                    for (int c4 = 0; c4 < 2; ++c4) {
                        u32x4 o;
#pragma unroll
                        for (int i = 0; i < 4; ++i) o[i] = pack2<F16>(val[0][4 * c4 + i], val[1][4 * c4 + i]);
                        *(u32x4 *)(drow + 8 * d + 4 * c4) = o;
                    }
                }
                if (S > 0) {
                    // salient values of tiles 2 m, 2 m + 1: codes 16 hi + lo with the
                    // payload as A operand, so lane (source gl, ql) gets tokens
                    // 4 ql + r, exactly the k-slot pairs of the P^T operand
                    float sv[2][4];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        i32x4 lo4, hi4;
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            lo4[d] = (int)(vk[2 * m + u][d] & 0x0f0f0f0fu);
                            hi4[d] = (int)((vk[2 * m + u][d] >> 4) & 0x0f0f0f0fu);
                        }
                        i32x4 code = __builtin_amdgcn_mfma_i32_16x16x64_i8(lo4, vsel_e, i32x4{0, 0, 0, 0}, 0, 0, 0);
                        code = __builtin_amdgcn_mfma_i32_16x16x64_i8(hi4, vsel_o, code, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; ++r) sv[u][r] = fmaf((float)code[r], vsf.x, vsf.y);
                    }
                    u32x4 sa;
#pragma unroll
                    for (int r = 0; r < 4; ++r) sa[r] = pack2<F16>(sv[0][r], sv[1][r]);
                    acc_sal = mma32<F16>(sa, phi[m], acc_sal);
                    acc_sal = mma32<F16>(sa, plo[m], acc_sal);
                }
            } else if (packed) {
                float s9[2], of[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    s9[u] = iq_f16_to_f32(vp[m][u][0]) * inv_unit;
                    of[u] = iq_f16_to_f32(vp[m][u][1]);
                }
                if constexpr (VBITS == 2) {
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
                            for (int i = 0; i < 4; ++i) o[i] = pack2<F16>(val[0][4 * c4 + i], val[1][4 * c4 + i]);
                            *(u32x4 *)(dst + 16 * w + 4 * c4) = o;
                        }
                    }
                } else {
#pragma unroll
                    for (int w = 0; w < 4; ++w) {          // 8 channels 32 qq + 8 w + (2 b + {0, 1})
                        float val[2][8];
#pragma unroll
                        for (int u = 0; u < 2; ++u) {
                            const uint32_t x = vw[m][u][w];
                            const uint32_t lo = x & 0x0f0f0f0fu, hi = (x >> 4) & 0x0f0f0f0fu;
                            const f32x2 e01 = fp8x2<false>(lo), e23 = fp8x2<true>(lo);
                            const f32x2 o01 = fp8x2<false>(hi), o23 = fp8x2<true>(hi);
                            val[u][0] = fmaf(e01.x, s9[u], of[u]);
                            val[u][1] = fmaf(o01.x, s9[u], of[u]);
                            val[u][2] = fmaf(e01.y, s9[u], of[u]);
                            val[u][3] = fmaf(o01.y, s9[u], of[u]);
                            val[u][4] = fmaf(e23.x, s9[u], of[u]);
                            val[u][5] = fmaf(o23.x, s9[u], of[u]);
                            val[u][6] = fmaf(e23.y, s9[u], of[u]);
                            val[u][7] = fmaf(o23.y, s9[u], of[u]);
                        }
#pragma unroll
                        for (int c4 = 0; c4 < 2; ++c4) {
                            u32x4 o;
#pragma unroll
                            for (int i = 0; i < 4; ++i) o[i] = pack2<F16>(val[0][4 * c4 + i], val[1][4 * c4 + i]);
                            *(u32x4 *)(dst + 8 * w + 4 * c4) = o;
                        }
                    }
                }
            } else {
                const int t0 = base + 32 * m + pl, t1 = t0 + 16;
                const int ta = t0 < stop ? t0 : stop - 1, tb = t1 < stop ? t1 : stop - 1;
                u32x4 r0[4], r1[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    r0[i] = ld16(dense_v(ta) + 32 * qq + 8 * i);
                    r1[i] = ld16(dense_v(tb) + 32 * qq + 8 * i);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (t0 >= stop) r0[i] = u32x4{0u, 0u, 0u, 0u};
                    if (t1 >= stop) r1[i] = u32x4{0u, 0u, 0u, 0u};
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
            // two row blocks at a time, so that consecutive products go to
            // different accumulators
#pragma unroll
            for (int n = 0; n < 8; n += 2) {
                u32x4 va[2];                           // k-slot pair r: pair row 4 ql + r
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int r = 0; r < 4; ++r) va[u][r] = vtile[(4 * ql + r) * VR + 16 * (n + u) + gl];
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    acc[n + u] = mma32<F16>(va[u], phi[m], m == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : acc[n + u]);
#pragma unroll
                for (int u = 0; u < 2; ++u) acc[n + u] = mma32<F16>(va[u], plo[m], acc[n + u]);
            }
        }
    } else {
#pragma unroll
        for (int n = 0; n < 8; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#undef IQ_LOAD_CHUNK

    if (PACKED || !a.dense_first) __builtin_amdgcn_s_setprio(1);
    // ---------------- combine the four wavefronts, write this partition's partial
    // Each wavefront stages its unnormalized O as O[g][c] rows next to its
    // (m, l); a reader weights the four rows by 2^(m_w - max m) and adds.
    l_run = xsum16(l_run);
    if (ql == 0) {
        s_wm[wave][gl] = m_run;
        s_wl[wave][gl] = l_run;
    }
    float *ot = (float *)vt;
#pragma unroll
    for (int n = 0; n < 8; ++n) *(f32x4 *)(ot + gl * OROW + 16 * n + 4 * ql) = acc[n];
    if constexpr (PACKED && K4V) {
        // the value columns that decoded to 0: a source's column takes its
        // 8-bit-code product, a donor's round(pad) * sum(p)
        if (S > 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int k = 4 * ql + e;
                if (k < S) {
                    ot[gl * OROW + sm.vsrc[k]] = acc_sal[e];
                    ot[gl * OROW + sm.vdon[k]] = sm.vdpad[k] * l_run;
                }
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < G * (D / 4); i += 256) {
        const int g = i >> 5, c = (i & 31) * 4;
        float mw[WAVES], mx = NEG_INF;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            mw[w] = s_wm[w][g];
            mx = fmaxf(mx, mw[w]);
        }
        f32x4 num = {0.0f, 0.0f, 0.0f, 0.0f};
        float den = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float wt = mw[w] == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - mx);
            const f32x4 o = *(const f32x4 *)((const float *)s_v[w] + g * OROW + c);
#pragma unroll
            for (int e = 0; e < 4; ++e) num[e] = fmaf(o[e], wt, num[e]);
            den = fmaf(s_wl[w][g], wt, den);
        }
        if (a.P == 1) {
#pragma unroll
            for (int e = 0; e < 4; ++e) iq_store_as(a.out, (int64_t)(h * G + g) * D + c + e, num[e] / den, a.odt);
            continue;
        }
        const Partials pt = partials(a.ws, a.H * G * a.P);
        const int64_t row = (int64_t)(h * G + g) * a.P + p;
        *(f32x4 *)(pt.o + row * D + c) = num;
        if (c == 0) pt.ml[row] = f32x2{mx * LN2, den};
    }
}

// K4-coded values keep twice the value payload and their own selection
// operands in registers: with fp16 queries three workgroups per compute
// unit instead of four (four would spill); bf16 fits four.
template <bool F16, int VBITS>
__global__ __launch_bounds__(256, VBITS == 0 && F16 ? 3 : 4) void decode_fast(FastArgs a)
{
    __shared__ FastSmem sm;
    if (partition_of(a, blockIdx.y) < a.nblk) fast_body<F16, VBITS, true>(a, sm);
    else fast_body<F16, VBITS, false>(a, sm);
}

// Workgroups of decode_fast<F16, VBITS> resident on the current device at
// once (compute units x occupancy), measured once per device; 0 if unknown.
template <bool F16, int VBITS>
int64_t resident_workgroups()
{
    static std::atomic<int64_t> cap[64];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int64_t c = cap[dev].load(std::memory_order_relaxed);
    if (c == 0) {
        int cus = 0, per = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, decode_fast<F16, VBITS>, 256, 0) != hipSuccess)
            return 0;
        c = (int64_t)cus * per;
        cap[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

}  // namespace

#undef IQ_LOAD_CHUNK

// Launches the matrix-core decode; returns IQ_ERR_UNSUPPORTED for layouts it
// does not cover.  Partitions are the packed blocks, then 32-token slices of
// sink ++ tail; *parts receives their count.  With one partition the output is
// written in-kernel, otherwise the caller merges *parts partials.
int iq_decode_fast_launch(const void *q, int q_dtype, int64_t q_stride_h, int64_t Hq, const int64_t *tables,
                          const int8_t *key_map, const int8_t *value_map, int64_t n_blocks, int64_t block_tokens,
                          int64_t H, int64_t S,
                          int value_bits, int value_group, const void *sink_k, const void *sink_v, int64_t sink_k_sh,
                          int64_t sink_k_st, int64_t sink_v_sh, int64_t sink_v_st, int64_t sink_t,
                          const void *tail_k, const void *tail_v, int64_t tail_k_sh, int64_t tail_k_st,
                          int64_t tail_v_sh, int64_t tail_v_st, int64_t tail_t, float scale, float *workspace,
                          void *out, int out_dtype, const iq_block_run *run, int64_t *parts, hipStream_t stream)
{
    if (q_dtype != IQ_BF16 && q_dtype != IQ_F16) return IQ_ERR_UNSUPPORTED;
    if (out_dtype != IQ_F32 && out_dtype != IQ_BF16 && out_dtype != IQ_F16) return IQ_ERR_UNSUPPORTED;
    if (n_blocks > 0 && value_bits != 0 && value_bits != 2 && value_bits != 4) return IQ_ERR_UNSUPPORTED;
    if (n_blocks > 0 && value_bits == 0 && !value_map) return IQ_ERR_UNSUPPORTED;
    if (n_blocks > 0 && value_bits != 0 && value_group != 32 && value_group != 64 && value_group != 128)
        return IQ_ERR_UNSUPPORTED;
    if (Hq / H > 16 || S > 16) return IQ_ERR_UNSUPPORTED;
    if (n_blocks > 0 && block_tokens > CHUNK * WAVES) return IQ_ERR_UNSUPPORTED;   // one pass per workgroup
    // query, dense rows and packed rows are read as 16-byte vectors
    auto aligned = [](const void *ptr, int64_t sh, int64_t st) {
        return ((uintptr_t)ptr % 16 == 0) && (sh % 8 == 0) && (st % 8 == 0);
    };
    if (!aligned(q, q_stride_h, 8)) return IQ_ERR_UNSUPPORTED;
    if (sink_t && !(aligned(sink_k, sink_k_sh, sink_k_st) && aligned(sink_v, sink_v_sh, sink_v_st)))
        return IQ_ERR_UNSUPPORTED;
    if (tail_t && !(aligned(tail_k, tail_k_sh, tail_k_st) && aligned(tail_v, tail_v_sh, tail_v_st)))
        return IQ_ERR_UNSUPPORTED;
    const int64_t P = n_blocks + (sink_t + tail_t + DENSE_SPLIT - 1) / DENSE_SPLIT;
    if (P < 1 || P > 65535) return IQ_ERR_UNSUPPORTED;
    FastArgs a{{}, 0, (const uint16_t *)q, q_stride_h, (int)(Hq / H), tables, key_map, value_map, n_blocks,
               block_tokens, H, S,
               value_group == 32 ? 5 : value_group == 128 ? 7 : 6, (const uint16_t *)sink_k, (const uint16_t *)sink_v, sink_k_sh,
               sink_k_st, sink_v_sh, sink_v_st, sink_t, (const uint16_t *)tail_k, (const uint16_t *)tail_v,
               tail_k_sh, tail_k_st, tail_v_sh, tail_v_st, tail_t, scale * 1.44269504088896341f, workspace, P,
               out, out_dtype};
    if (run && run->blocks > 0 && n_blocks > 0) {
        for (int k = 0; k < IQ_TABLE_COLS; ++k) a.run[k] = (const uint8_t *)run->base[k];
        a.run_blocks = run->blocks < n_blocks ? run->blocks : n_blocks;
    }
    *parts = P;
    const dim3 grid((unsigned)H, (unsigned)P), block(256);
    const bool f16 = q_dtype == IQ_F16;
    const int vb = n_blocks > 0 ? value_bits : 2;
    if (n_blocks > 0 && P > n_blocks) {
        const int64_t cap = f16 ? (vb == 2 ? resident_workgroups<true, 2>() : vb == 4 ? resident_workgroups<true, 4>()
                                                                                      : resident_workgroups<true, 0>())
                                : (vb == 2 ? resident_workgroups<false, 2>() : vb == 4 ? resident_workgroups<false, 4>()
                                                                                       : resident_workgroups<false, 0>());
        a.dense_first = cap > 0 && H * P > cap;
    }
    if (f16 && vb == 2) hipLaunchKernelGGL((decode_fast<true, 2>), grid, block, 0, stream, a);
    else if (f16 && vb == 4) hipLaunchKernelGGL((decode_fast<true, 4>), grid, block, 0, stream, a);
    else if (f16) hipLaunchKernelGGL((decode_fast<true, 0>), grid, block, 0, stream, a);
    else if (vb == 2) hipLaunchKernelGGL((decode_fast<false, 2>), grid, block, 0, stream, a);
    else if (vb == 4) hipLaunchKernelGGL((decode_fast<false, 4>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((decode_fast<false, 0>), grid, block, 0, stream, a);
    return IQ_OK;
}
