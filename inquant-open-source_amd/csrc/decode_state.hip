// Incremental decode-metadata append (gfx950).
//
// Restates PackedDecodeState.extend / _write_maps (triton_attention.py:234-309):
// for each newly sealed block, one row of the i64 pointer table
// (K payload, K scales, K padding, V payload, V scales-or-K4-scales,
// V offsets-or-padding, then the K source and donor descriptor addresses
// that the decode kernel reads directly) and an int8 [H, 128] role map per coded tensor:
// -1 normal, donor channel for a source, -2 - i for donor i.
// The block addresses travel as kernel arguments, so no host-to-device copy
// of a pageable pointer list is needed.
#include "iq_common.h"

namespace {

constexpr int APPEND_CHUNK = 24;       // blocks per launch (kernel-argument budget)

// N block address rows travel as kernel arguments: N = 1 for the usual
// one-block append of a seal (~140 argument bytes to write at launch, not ~2 KB)
template <int N>
struct AppendArgs {
    int64_t *tables;
    int8_t *key_map, *value_map;
    int64_t first, count, H, S;
    int desc_bytes;
    iq_block_ptrs blocks[N];
};

__device__ __forceinline__ int load_desc(uint64_t p, int64_t i, int bytes)
{
    if (bytes == 1) return ((const uint8_t *)p)[i];
    if (bytes == 4) return ((const int32_t *)p)[i];
    return (int)((const int64_t *)p)[i];
}

// grid (count, H): one 128-thread workgroup writes one block's map for one head.
template <int N>
__global__ __launch_bounds__(128) void append_kernel(AppendArgs<N> a)
{
    __shared__ int8_t s_k[128], s_v[128];
    const int blk = blockIdx.x, h = blockIdx.y, c = threadIdx.x;
    const iq_block_ptrs &p = a.blocks[blk];
    const int64_t slot = a.first + blk;
    if (h == 0 && c < IQ_TABLE_COLS) {
        const uint64_t v[IQ_TABLE_COLS] = {p.k_payload, p.k_scales, p.k_padding, p.v_payload,
                                           p.v_scales,  p.v_offsets, p.k_src, p.k_don};
        a.tables[slot * IQ_TABLE_COLS + c] = (int64_t)v[c];
    }
    s_k[c] = -1;
    s_v[c] = -1;
    __syncthreads();
    if (c < a.S) {
        const int s = load_desc(p.k_src, h * a.S + c, a.desc_bytes);
        s_k[s] = (int8_t)load_desc(p.k_don, h * a.S + c, a.desc_bytes);
        if (a.value_map) s_v[load_desc(p.v_src, h * a.S + c, a.desc_bytes)] =
            (int8_t)load_desc(p.v_don, h * a.S + c, a.desc_bytes);
    }
    __syncthreads();
    if (c < a.S) {
        s_k[load_desc(p.k_don, h * a.S + c, a.desc_bytes)] = (int8_t)(-2 - c);
        if (a.value_map) s_v[load_desc(p.v_don, h * a.S + c, a.desc_bytes)] = (int8_t)(-2 - c);
    }
    __syncthreads();
    a.key_map[(slot * a.H + h) * 128 + c] = s_k[c];
    if (a.value_map) a.value_map[(slot * a.H + h) * 128 + c] = s_v[c];
}

template <int N>
int launch_append(int64_t *tables, int8_t *key_map, int8_t *value_map, int64_t first, int64_t n,
                  const iq_block_ptrs *blocks, int64_t H, int64_t S, int desc_bytes, void *stream)
{
    AppendArgs<N> a{};
    a.tables = tables;
    a.key_map = key_map;
    a.value_map = value_map;
    a.first = first;
    a.count = n;
    a.H = H;
    a.S = S;
    a.desc_bytes = desc_bytes;
    for (int64_t i = 0; i < n; ++i) a.blocks[i] = blocks[i];
    hipLaunchKernelGGL(append_kernel<N>, dim3((unsigned)n, (unsigned)H), dim3(128), 0, (hipStream_t)stream, a);
    IQ_CHECK_LAUNCH("append_kernel");
    return IQ_OK;
}

}  // namespace

extern "C" int iq_decode_append(int64_t *tables, int8_t *key_map, int8_t *value_map, int64_t first,
                                int64_t count, const iq_block_ptrs *blocks, int64_t H, int64_t S, int desc_bytes,
                                void *stream)
{
    IQ_CHECK_ARG(first >= 0 && count >= 0, "iq_decode_append: bad range");
    if (count == 0) return IQ_OK;
    IQ_CHECK_ARG(tables && key_map && blocks, "iq_decode_append: null pointer");
    IQ_CHECK_ARG(H >= 1 && H <= 65535, "iq_decode_append: bad H");
    IQ_CHECK_ARG(S >= 0 && S <= 64, "iq_decode_append: S=%lld must be <= 64 (int8 roles, D = 128)", (long long)S);
    IQ_CHECK_ARG(desc_bytes == 1 || desc_bytes == 4 || desc_bytes == 8, "iq_decode_append: desc_bytes");
    for (int64_t i = 0; i < count; ++i) {
        IQ_CHECK_ARG(blocks[i].k_payload && blocks[i].k_scales && blocks[i].v_payload && blocks[i].v_scales,
                     "iq_decode_append: block %lld has a null address", (long long)i);
        IQ_CHECK_ARG(S == 0 || (blocks[i].k_src && blocks[i].k_don), "iq_decode_append: missing K descriptors");
        IQ_CHECK_ARG(!value_map || S == 0 || (blocks[i].v_src && blocks[i].v_don),
                     "iq_decode_append: missing V descriptors");
    }
    if (count == 1) return launch_append<1>(tables, key_map, value_map, first, 1, blocks, H, S, desc_bytes, stream);
    for (int64_t done = 0; done < count; done += APPEND_CHUNK) {
        const int64_t n = count - done < APPEND_CHUNK ? count - done : APPEND_CHUNK;
        const int rc = launch_append<APPEND_CHUNK>(tables, key_map, value_map, first + done, n, blocks + done, H, S,
                                                   desc_bytes, stream);
        if (rc != IQ_OK) return rc;
    }
    return IQ_OK;
}
