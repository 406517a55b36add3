// In-place append of dense tokens to a cache layer's recent tail (gfx950).
//
// The reference's cache concatenates the whole dense tail with every new
// token (cache.py:256-259 and :283-286: two torch.cat of up to R + B - 1
// rows per layer per token).  Here the tail lives in a preallocated
// [2 (keys, values), H, capacity, D] buffer and one launch:
//   * moves `shift_count` rows from `shift_src` down to row 0 (the rows that
//     survive a seal: the sealed block's rows are dropped by moving the
//     survivors, once, at the first append after the seal);
//   * writes the n_new new rows at `slot`;
//   * compares the caller's cache_position values with expected + i and
//     sets *flag on a mismatch (the host reads the flag where it
//     synchronizes anyway; rows past the live tail are scratch, so a token
//     written under a bad position is simply not counted).
// Rows are copied with 16-byte vector loads and stores when every address
// and stride allows it, else 4- or 2-byte units.
#include "iq_common.h"

namespace {

struct TailArgs {
    const char *k, *v;                 // new rows, byte strides (head, token)
    int64_t k_sh, k_st, v_sh, v_st;
    char *buf;                         // [2, H, capacity, D] byte strides
    int64_t b_kv, b_h, b_t;
    int64_t H, n_new, row_units;
    int64_t slot, shift_src, shift_count;
    const void *pos;
    int pos_bytes;
    int64_t expected;
    int *flag;
};

// grid.x = (n_new + shift_count) * H rows, grid.y = 2 (keys, values)
template <typename U>
__global__ __launch_bounds__(64) void tail_append_kernel(TailArgs a)
{
    const int64_t r = blockIdx.x;
    const int kv = blockIdx.y;
    const int64_t h = r % a.H, t = r / a.H;
    const char *src;
    char *dst = a.buf + kv * a.b_kv + h * a.b_h;
    if (t < a.n_new) {
        src = kv ? a.v + h * a.v_sh + t * a.v_st : a.k + h * a.k_sh + t * a.k_st;
        dst += (a.slot + t) * a.b_t;
    } else {
        const int64_t s = t - a.n_new;
        src = a.buf + kv * a.b_kv + h * a.b_h + (a.shift_src + s) * a.b_t;
        dst += s * a.b_t;
    }
    for (int64_t i = threadIdx.x; i < a.row_units; i += 64) ((U *)dst)[i] = ((const U *)src)[i];
    if (r == 0 && kv == 0 && a.pos && threadIdx.x < a.n_new) {
        const int64_t i = threadIdx.x;
        const int64_t got = a.pos_bytes == 8 ? ((const int64_t *)a.pos)[i] : (int64_t)((const int32_t *)a.pos)[i];
        if (got != a.expected + i) *a.flag = 1;
    }
}

}  // namespace

extern "C" int iq_tail_append(const void *k, const void *v, int64_t k_sh, int64_t k_st, int64_t v_sh, int64_t v_st,
                              int64_t H, int64_t n_new, int64_t D, int elem_bytes, void *buf, int64_t buf_kv,
                              int64_t buf_h, int64_t buf_t, int64_t capacity, int64_t slot, int64_t shift_src,
                              int64_t shift_count, const void *positions, int pos_bytes, int64_t expected, int *flag,
                              void *stream)
{
    IQ_CHECK_ARG(buf && H >= 1 && D >= 1 && n_new >= 0 && shift_count >= 0, "iq_tail_append: bad arguments");
    IQ_CHECK_ARG(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
                 "iq_tail_append: element size %d", elem_bytes);
    IQ_CHECK_ARG(n_new == 0 || (k && v), "iq_tail_append: null key/value rows");
    IQ_CHECK_ARG(n_new <= 64, "iq_tail_append: at most 64 new rows per call");
    IQ_CHECK_ARG(slot >= 0 && slot + n_new <= capacity, "iq_tail_append: rows [%lld, %lld) outside capacity %lld",
                 (long long)slot, (long long)(slot + n_new), (long long)capacity);
    if (shift_count > 0) {
        // source, destination and new rows must be disjoint (no ordering inside the launch)
        IQ_CHECK_ARG(shift_src >= shift_count && shift_src + shift_count <= capacity,
                     "iq_tail_append: overlapping or out-of-range move");
        IQ_CHECK_ARG(slot >= shift_count && (slot + n_new <= shift_src || slot >= shift_src + shift_count),
                     "iq_tail_append: new rows overlap the moved rows");
    }
    IQ_CHECK_ARG(!positions || ((pos_bytes == 4 || pos_bytes == 8) && flag), "iq_tail_append: bad position check");
    IQ_CHECK_ARG(H * (n_new + shift_count) <= 0x7fffffffLL, "iq_tail_append: too many rows");
    if (n_new + shift_count == 0) return IQ_OK;
    const int64_t row_bytes = D * elem_bytes;
    const int64_t eb = elem_bytes;
    const int64_t byte_strides[7] = {k_sh * eb, k_st * eb, v_sh * eb, v_st * eb, buf_kv * eb, buf_h * eb, buf_t * eb};
    auto fits = [&](int64_t unit) {
        if (row_bytes % unit) return false;
        if ((uintptr_t)buf % unit || (n_new && ((uintptr_t)k % unit || (uintptr_t)v % unit))) return false;
        for (int64_t s : byte_strides)
            if (s % unit) return false;
        return true;
    };
    TailArgs a{(const char *)k, (const char *)v, byte_strides[0], byte_strides[1], byte_strides[2], byte_strides[3],
               (char *)buf, byte_strides[4], byte_strides[5], byte_strides[6], H, n_new, 0, slot, shift_src,
               shift_count, positions, pos_bytes, expected, flag};
    const dim3 grid((unsigned)(H * (n_new + shift_count)), 2), block(64);
    hipStream_t s = (hipStream_t)stream;
    if (fits(16)) {
        a.row_units = row_bytes / 16;
        hipLaunchKernelGGL(tail_append_kernel<uint4>, grid, block, 0, s, a);
    } else if (fits(4)) {
        a.row_units = row_bytes / 4;
        hipLaunchKernelGGL(tail_append_kernel<uint32_t>, grid, block, 0, s, a);
    } else if (fits(2)) {
        a.row_units = row_bytes / 2;
        hipLaunchKernelGGL(tail_append_kernel<uint16_t>, grid, block, 0, s, a);
    } else {
        a.row_units = row_bytes;
        hipLaunchKernelGGL(tail_append_kernel<uint8_t>, grid, block, 0, s, a);
    }
    IQ_CHECK_LAUNCH("tail_append_kernel");
    return IQ_OK;
}

extern "C" int iq_tail_append_row(const iq_tail_desc *d, const void *k, const void *v, int64_t slot,
                                  int64_t shift_src, int64_t shift_count, const void *positions, int64_t expected,
                                  void *stream)
{
    IQ_CHECK_ARG(d, "iq_tail_append_row: null descriptor");
    return iq_tail_append(k, v, d->k_sh, d->k_st, d->v_sh, d->v_st, d->heads, 1, d->dim, d->elem_bytes,
                          (void *)d->buf, d->buf_kv, d->buf_h, d->buf_t, d->capacity, slot, shift_src, shift_count,
                          positions, d->pos_bytes, expected, (int *)d->flag, stream);
}
