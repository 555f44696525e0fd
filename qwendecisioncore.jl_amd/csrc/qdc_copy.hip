// qdc_copy.hip -- a plain device copy in the streaming shape the row kernels
// use at their best: one 16-byte chunk per thread, nontemporal load and store,
// no arithmetic.  It has no counterpart in the reference.  A single launch of
// this copy at a given byte count is the practical bandwidth ceiling that a
// row kernel moving the same bytes can be held against (launch ramp-up and
// drain included), so the benchmark times it beside each kernel.
#include "qdc_common.hpp"

namespace qdc {
namespace {

__global__ __launch_bounds__(kBlock) void copy_chunks(u32x4 *__restrict__ dst,
                                                      const u32x4 *__restrict__ src, uint32_t n) {
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i < n) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// chunks * 16 bytes; the grid (chunks rounded up to whole workgroups) stays
// below 2^32 work-items
constexpr int64_t kMaxChunks = ((int64_t)1 << 32) - kBlock;

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
