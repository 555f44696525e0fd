// qdc_copy.hip -- plain device copies in the streaming shape the row kernels
// use at their best: one 16-byte chunk per thread, nontemporal load and store,
// no arithmetic.  Neither has a counterpart in the reference.  A single launch
// of qdc_copy at a given byte count is the practical bandwidth ceiling that a
// row kernel moving the same bytes can be held against (launch ramp-up and
// drain included), so the benchmark times it beside each kernel; qdc_copy_rows
// is the same for the embedding gather's access pattern (whole rows read at
// random places of a large table, written contiguously), and qdc_empty the
// fixed cost of a launch of a given grid (workgroups that do nothing).
#include "qdc_common.hpp"

namespace qdc {
namespace {

__global__ __launch_bounds__(kBlock) void copy_chunks(u32x4 *__restrict__ dst,
                                                      const u32x4 *__restrict__ src, uint32_t n) {
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i < n) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// CPT chunks per thread: workgroup b covers chunks [b*CPT*BLOCK, (b+1)*CPT*BLOCK),
// the k-th load instruction of every thread the k-th run of BLOCK consecutive
// chunks, so each wavefront instruction stays one contiguous 1 KB span; all
// loads are issued before the first store.
// A workgroup wholly inside the buffer (every one but the last, in general)
// takes the unguarded form, so no load or store sits in a branch of its own.
template <int CPT, int BLOCK>
__global__ __launch_bounds__(BLOCK) void copy_grid(u32x4 *__restrict__ dst,
                                                   const u32x4 *__restrict__ src, uint32_t n) {
    const uint32_t first = blockIdx.x * (CPT * BLOCK), base = first + threadIdx.x;
    u32x4 v[CPT];
    if (first + CPT * BLOCK <= n) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) v[k] = __builtin_nontemporal_load(src + base + k * BLOCK);
#pragma unroll
        for (int k = 0; k < CPT; ++k) __builtin_nontemporal_store(v[k], dst + base + k * BLOCK);
        return;
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k)
        if (base + k * BLOCK < n) v[k] = __builtin_nontemporal_load(src + base + k * BLOCK);
#pragma unroll
    for (int k = 0; k < CPT; ++k)
        if (base + k * BLOCK < n) __builtin_nontemporal_store(v[k], dst + base + k * BLOCK);
}

// Two copies in one launch: thread t copies chunk t (and t + BLOCK, ... for CPT
// chunks, as copy_grid) of stream 0 and of stream 1 where they exist: all of
// stream 0's loads, then stream 1's, then the stores in the same order (the
// faster of the two orders measured; the residual norm loads the same way).
// The access structure of a row kernel that reads two tensors and writes two.
template <int CPT, int BLOCK>
__global__ __launch_bounds__(BLOCK) void copy_pair(u32x4 *__restrict__ d0,
                                                   const u32x4 *__restrict__ s0, uint32_t n0,
                                                   u32x4 *__restrict__ d1,
                                                   const u32x4 *__restrict__ s1, uint32_t n1) {
    const uint32_t first = blockIdx.x * (CPT * BLOCK), base = first + threadIdx.x;
    u32x4 a[CPT], b[CPT];
    if (first + CPT * BLOCK <= n0 && first + CPT * BLOCK <= n1) {  // wholly inside both
#pragma unroll
        for (int k = 0; k < CPT; ++k) a[k] = __builtin_nontemporal_load(s0 + base + k * BLOCK);
#pragma unroll
        for (int k = 0; k < CPT; ++k) b[k] = __builtin_nontemporal_load(s1 + base + k * BLOCK);
#pragma unroll
        for (int k = 0; k < CPT; ++k) __builtin_nontemporal_store(a[k], d0 + base + k * BLOCK);
#pragma unroll
        for (int k = 0; k < CPT; ++k) __builtin_nontemporal_store(b[k], d1 + base + k * BLOCK);
        return;
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k)
        if (base + k * BLOCK < n0) a[k] = __builtin_nontemporal_load(s0 + base + k * BLOCK);
#pragma unroll
    for (int k = 0; k < CPT; ++k)
        if (base + k * BLOCK < n1) b[k] = __builtin_nontemporal_load(s1 + base + k * BLOCK);
#pragma unroll
    for (int k = 0; k < CPT; ++k)
        if (base + k * BLOCK < n0) __builtin_nontemporal_store(a[k], d0 + base + k * BLOCK);
#pragma unroll
    for (int k = 0; k < CPT; ++k)
        if (base + k * BLOCK < n1) __builtin_nontemporal_store(b[k], d1 + base + k * BLOCK);
}

// chunks * 16 bytes; the grid (chunks rounded up to whole workgroups) stays
// below 2^32 work-items
constexpr int64_t kMaxChunks = ((int64_t)1 << 32) - 8 * 512;

// An empty workgroup: the fixed cost of a launch of a given grid.
__global__ __launch_bounds__(kBlock) void empty_grid() {}

// Random-row copy: thread g copies 16-byte chunk c of source row rows[i]
// (g = i * chunks + c) into each of the `repeat` copies of destination row i.
// A store instruction of a wavefront writes one contiguous span per copy.  A
// row index outside [0, n_src) copies nothing and writes zeros.
template <int REPEAT>
__global__ __launch_bounds__(kBlock) void copy_rows(u32x4 *__restrict__ dst,
                                                    const u32x4 *__restrict__ src,
                                                    const int32_t *__restrict__ rows,
                                                    uint32_t total, FastDiv chunks,
                                                    int64_t n_src) {
    const uint32_t g = blockIdx.x * kBlock + threadIdx.x;
    if (g >= total) return;
    const uint32_t i = fastdiv(g, chunks);
    const uint32_t c = g - i * chunks.d;
    const int64_t r = rows[i];
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r >= 0 && r < n_src) v = __builtin_nontemporal_load(src + r * chunks.d + c);
    u32x4 *d = dst + (int64_t)i * chunks.d * REPEAT + c;
#pragma unroll
    for (int k = 0; k < REPEAT; ++k) __builtin_nontemporal_store(v, d + k * (int64_t)chunks.d);
}

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" int32_t qdc_copy(void *dst, const void *src, int64_t bytes, hipStream_t stream) {
    if (bytes < 0 || bytes % 16 != 0 || bytes / 16 > kMaxChunks) return QDC_ERR_SHAPE;
    if (bytes == 0) return QDC_OK;
    if (!dst || !src) return QDC_ERR_NULL;
    if (!aligned16(dst) || !aligned16(src)) return QDC_ERR_SHAPE;
    if (overlaps(dst, bytes, src, bytes)) return QDC_ERR_ALIAS;
    const int64_t n = bytes / 16;
    hipLaunchKernelGGL(copy_chunks, dim3((uint32_t)ceil_div(n, kBlock)), dim3(kBlock), 0, stream,
                       static_cast<u32x4 *>(dst), static_cast<const u32x4 *>(src), (uint32_t)n);
    return launch_status();
}

extern "C" int32_t qdc_copy_grid(void *dst, const void *src, int64_t bytes,
                                 int32_t chunks_per_thread, int32_t block, hipStream_t stream) {
    if (bytes < 0 || bytes % 16 != 0 || bytes / 16 > kMaxChunks) return QDC_ERR_SHAPE;
    if (block != 256 && block != 512) return QDC_ERR_SHAPE;
    if (chunks_per_thread != 1 && chunks_per_thread != 2 && chunks_per_thread != 4 &&
        chunks_per_thread != 8)
        return QDC_ERR_SHAPE;
    if (bytes == 0) return QDC_OK;
    if (!dst || !src) return QDC_ERR_NULL;
    if (!aligned16(dst) || !aligned16(src)) return QDC_ERR_SHAPE;
    if (overlaps(dst, bytes, src, bytes)) return QDC_ERR_ALIAS;
    const int64_t n = bytes / 16;
    const dim3 grid((uint32_t)ceil_div(n, (int64_t)chunks_per_thread * block));
    auto *d = static_cast<u32x4 *>(dst);
    auto *s = static_cast<const u32x4 *>(src);
#define QDC_COPY_GRID(C, B)                                                                      \
    if (chunks_per_thread == C && block == B) {                                                  \
        hipLaunchKernelGGL((copy_grid<C, B>), grid, dim3(B), 0, stream, d, s, (uint32_t)n);      \
        return launch_status();                                                                  \
    }
    QDC_COPY_GRID(1, 256)
    QDC_COPY_GRID(2, 256)
    QDC_COPY_GRID(4, 256)
    QDC_COPY_GRID(8, 256)
    QDC_COPY_GRID(1, 512)
    QDC_COPY_GRID(2, 512)
    QDC_COPY_GRID(4, 512)
    QDC_COPY_GRID(8, 512)
#undef QDC_COPY_GRID
    return QDC_ERR_SHAPE;
}

extern "C" int32_t qdc_copy_pair(void *dst0, const void *src0, int64_t bytes0, void *dst1,
                                 const void *src1, int64_t bytes1, int32_t chunks_per_thread,
                                 int32_t block, hipStream_t stream) {
    for (const int64_t b : {bytes0, bytes1})
        if (b < 0 || b % 16 != 0 || b / 16 > kMaxChunks) return QDC_ERR_SHAPE;
    if (block != 256 && block != 512) return QDC_ERR_SHAPE;
    if (chunks_per_thread != 1 && chunks_per_thread != 2 && chunks_per_thread != 4 &&
        chunks_per_thread != 8)
        return QDC_ERR_SHAPE;
    if (bytes0 == 0 && bytes1 == 0) return QDC_OK;
    if ((bytes0 && (!dst0 || !src0)) || (bytes1 && (!dst1 || !src1))) return QDC_ERR_NULL;
    if ((bytes0 && (!aligned16(dst0) || !aligned16(src0))) ||
        (bytes1 && (!aligned16(dst1) || !aligned16(src1))))
        return QDC_ERR_SHAPE;
    // each destination overlaps neither source nor the other destination
    if (overlaps(dst0, bytes0, src0, bytes0) || overlaps(dst0, bytes0, src1, bytes1) ||
        overlaps(dst1, bytes1, src0, bytes0) || overlaps(dst1, bytes1, src1, bytes1) ||
        overlaps(dst0, bytes0, dst1, bytes1))
        return QDC_ERR_ALIAS;
    const int64_t n0 = bytes0 / 16, n1 = bytes1 / 16;
    const dim3 grid((uint32_t)ceil_div(std::max(n0, n1), (int64_t)chunks_per_thread * block));
    auto *d0 = static_cast<u32x4 *>(dst0);
    auto *d1 = static_cast<u32x4 *>(dst1);
    auto *s0 = static_cast<const u32x4 *>(src0);
    auto *s1 = static_cast<const u32x4 *>(src1);
#define QDC_COPY_PAIR(C, B)                                                                      \
    if (chunks_per_thread == C && block == B) {                                                  \
        hipLaunchKernelGGL((copy_pair<C, B>), grid, dim3(B), 0, stream, d0, s0, (uint32_t)n0,    \
                           d1, s1, (uint32_t)n1);                                                \
        return launch_status();                                                                  \
    }
    QDC_COPY_PAIR(1, 256)
    QDC_COPY_PAIR(2, 256)
    QDC_COPY_PAIR(4, 256)
    QDC_COPY_PAIR(8, 256)
    QDC_COPY_PAIR(1, 512)
    QDC_COPY_PAIR(2, 512)
    QDC_COPY_PAIR(4, 512)
    QDC_COPY_PAIR(8, 512)
#undef QDC_COPY_PAIR
    return QDC_ERR_SHAPE;
}

extern "C" int32_t qdc_copy_rows(void *dst, const void *src, const int32_t *rows, int64_t n_rows,
                                 int64_t n_src, int64_t row_bytes, int32_t repeat,
                                 hipStream_t stream) {
    if (n_rows < 0 || n_src < 0 || row_bytes < 0 || row_bytes % 16 != 0 || repeat < 1 ||
        repeat > 4)
        return QDC_ERR_SHAPE;
    const int64_t chunks = row_bytes / 16;
    if (n_rows * chunks >= ((int64_t)1 << 31)) return QDC_ERR_SHAPE;
    if (n_rows == 0 || chunks == 0) return QDC_OK;
    if (!dst || !src || !rows) return QDC_ERR_NULL;
    if (!aligned16(dst) || !aligned16(src)) return QDC_ERR_SHAPE;
    const int64_t out_bytes = n_rows * row_bytes * repeat;
    if (overlaps(dst, out_bytes, src, n_src * row_bytes) || overlaps(dst, out_bytes, rows, n_rows * 4))
        return QDC_ERR_ALIAS;
    const uint32_t total = (uint32_t)(n_rows * chunks);
    const dim3 grid((uint32_t)ceil_div(total, kBlock));
#define QDC_ROWS(R)                                                                        \
    if (repeat == R)                                                                       \
        hipLaunchKernelGGL(copy_rows<R>, grid, dim3(kBlock), 0, stream,                    \
                           static_cast<u32x4 *>(dst), static_cast<const u32x4 *>(src), rows, \
                           total, make_fastdiv((uint32_t)chunks), n_src);
    QDC_ROWS(1)
    QDC_ROWS(2)
    QDC_ROWS(3)
    QDC_ROWS(4)
#undef QDC_ROWS
    return launch_status();
}

extern "C" int32_t qdc_empty(int64_t workgroups, hipStream_t stream) {
    if (workgroups < 0 || workgroups >= ((int64_t)1 << 32) / kBlock) return QDC_ERR_SHAPE;
    if (workgroups == 0) return QDC_OK;
    hipLaunchKernelGGL(empty_grid, dim3((uint32_t)workgroups), dim3(kBlock), 0, stream);
    return launch_status();
}
