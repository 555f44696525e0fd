// qdc_common.hpp -- shared device helpers for the CDNA4 (gfx950) row kernels.
//
// Data moves in 16-byte chunks (global_load/store_dwordx4): 4 fp32 or 8 bf16
// values.  Arithmetic is fp32; bf16 is widened by a shift and narrowed with the
// hardware round-to-nearest-even pack (v_cvt_pk_bf16_f32), which equals the
// reference's RNE formula (src/safetensors.jl:37-42) on every finite value.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qdc_hip.h"

namespace qdc {

typedef uint16_t bf16_t;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kBlock = 256;  // 4 wavefronts per workgroup

template <typename T> struct Elem;
template <> struct Elem<float> {
    static constexpr int kVec = 4;  // elements per 16-byte chunk
};
template <> struct Elem<bf16_t> {
    static constexpr int kVec = 8;
};

// ---------------------------------------------------------------- scalars --
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) { return __uint_as_float((uint32_t)v << 16); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
    f32x2 p = {v, 0.0f};
    bf16x2 b = __builtin_convertvector(p, bf16x2);
    return (bf16_t)(__builtin_bit_cast(uint32_t, b) & 0xffffu);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    f32x2 p = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2));
}

// ------------------------------------------------------ 16-byte chunk I/O --
// A chunk is loaded as raw 16 bytes (one global_load_dwordx4) and unpacked to
// fp32 only where it is used; `p` must be 16-byte aligned.
__device__ __forceinline__ u32x4 load_raw(const void *p) {
    return *reinterpret_cast<const u32x4 *>(p);
}
// Outputs are written once and not read again by the same launch: a
// nontemporal store streams them out instead of parking dirty lines in L2
// (measured 3-5% faster than a plain store for 16-176 MB streams on gfx950).
__device__ __forceinline__ void store_raw(void *p, u32x4 r) {
    __builtin_nontemporal_store(r, reinterpret_cast<u32x4 *>(p));
}
// Streamed data read exactly once per launch: a nontemporal load, so it does
// not displace reused lines (weights, RoPE tables) in the caches.
__device__ __forceinline__ u32x4 load_stream(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

__device__ __forceinline__ void unpack(u32x4 r, float (&v)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(r[i]);
}
__device__ __forceinline__ void unpack(u32x4 r, float (&v)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(r[i] << 16);
        v[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
}
__device__ __forceinline__ u32x4 pack(const float (&v)[4]) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = __float_as_uint(v[i]);
    return r;
}
__device__ __forceinline__ u32x4 pack(const float (&v)[8]) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    return r;
}

__device__ __forceinline__ void load_chunk(const float *p, float (&v)[4]) { unpack(load_raw(p), v); }
__device__ __forceinline__ void load_chunk(const bf16_t *p, float (&v)[8]) { unpack(load_raw(p), v); }
__device__ __forceinline__ void store_chunk(float *p, const float (&v)[4]) { store_raw(p, pack(v)); }
__device__ __forceinline__ void store_chunk(bf16_t *p, const float (&v)[8]) { store_raw(p, pack(v)); }

// ----------------------------------------------- V-element fragments ---
// V consecutive elements of type T held as raw vectors: whole 16-byte chunks,
// or one 8-byte piece (4 bf16).  Lets one kernel mix fp32 and bf16 tensors at
// the same element granularity: at 4 elements per lane an fp32 tensor moves in
// 16-byte chunks and a bf16 tensor in 8-byte pieces, so every load or store
// instruction of a wavefront covers one contiguous span (8 elements per lane
// would split each fp32 group over two 16-byte accesses 32 bytes apart).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename T, int V> struct Frag {
    static constexpr int kBytes = V * (int)sizeof(T);
    static constexpr bool kHalf = kBytes == 8;  // one 8-byte piece in r[0].xy
    static constexpr int kN = kHalf ? 1 : kBytes / 16;
    static_assert(kHalf || (kN >= 1 && kN * 16 == kBytes),
                  "fragment must be an 8-byte piece or whole 16-byte chunks");
    u32x4 r[kN];
};

template <typename T, int V> __device__ __forceinline__ Frag<T, V> load_frag(const T *p) {
    Frag<T, V> f;
    if constexpr (Frag<T, V>::kHalf) {
        const u32x2 h = *reinterpret_cast<const u32x2 *>(p);
        f.r[0] = u32x4{h[0], h[1], 0u, 0u};
    } else {
#pragma unroll
        for (int i = 0; i < Frag<T, V>::kN; ++i) f.r[i] = load_raw(p + i * (16 / (int)sizeof(T)));
    }
    return f;
}
template <typename T, int V> __device__ __forceinline__ Frag<T, V> stream_frag(const T *p) {
    Frag<T, V> f;
    if constexpr (Frag<T, V>::kHalf) {
        const u32x2 h = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
        f.r[0] = u32x4{h[0], h[1], 0u, 0u};
    } else {
#pragma unroll
        for (int i = 0; i < Frag<T, V>::kN; ++i) f.r[i] = load_stream(p + i * (16 / (int)sizeof(T)));
    }
    return f;
}
template <int V> __device__ __forceinline__ void unpack(const Frag<float, V> &f, float (&v)[V]) {
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = __uint_as_float(f.r[i / 4][i % 4]);
}
template <int V> __device__ __forceinline__ void unpack(const Frag<bf16_t, V> &f, float (&v)[V]) {
#pragma unroll
    for (int i = 0; i < V / 2; ++i) {
        const uint32_t b = f.r[i / 4][i % 4];
        v[2 * i] = __uint_as_float(b << 16);
        v[2 * i + 1] = __uint_as_float(b & 0xffff0000u);
    }
}
template <int V> __device__ __forceinline__ void store_frag(float *p, const float (&v)[V]) {
#pragma unroll
    for (int i = 0; i < V / 4; ++i) {
        u32x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = __float_as_uint(v[4 * i + e]);
        store_raw(p + 4 * i, r);
    }
}
template <int V> __device__ __forceinline__ void store_frag(bf16_t *p, const float (&v)[V]) {
    if constexpr (V == 4) {  // one 8-byte piece
        const u32x2 h = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        __builtin_nontemporal_store(h, reinterpret_cast<u32x2 *>(p));
    } else {
#pragma unroll
        for (int i = 0; i < V / 8; ++i) {
            u32x4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = pack_bf16x2(v[8 * i + 2 * e], v[8 * i + 2 * e + 1]);
            store_raw(p + 8 * i, r);
        }
    }
}

// ------------------------------------------------------ two-term bf16 ----
// The split output form (QDC_BF16X2): an fp32 value v is written as two bf16
// terms, hi = bf16(v) and lo = bf16(v - hi) (both round to nearest even), so
// hi + lo keeps about 16 significant bits (|v - (hi + lo)| <= 2^-17 |v| for
// normal v: |v - hi| <= 2^-8 |v| and lo rounds that rest to 8 bits).  A
// non-finite hi (inf, NaN, or v beyond the bf16 range) gets lo = 0.  Element e
// of a split tensor takes bf16 slots 8*(e/4) + e%4 (hi) and 8*(e/4) + 4 + e%4
// (lo): each aligned group of 4 elements is one 16-byte piece [4 hi | 4 lo], so
// a split element has the 4-byte footprint of an fp32 one and every address
// computation of an fp32 output applies unchanged.  A GEMM reads a split row
// of K elements as 2K bf16 values against a weight whose K rows are repeated
// in the same pattern: sum(hi*w + lo*w) = sum((hi + lo)*w) with bf16 operands.
struct split_t {
    uint32_t bits;
};

// Tensors a kernel reads beside a split output (norm weights, gates) are bf16.
template <typename T> struct AuxOf {
    typedef T type;
};
template <> struct AuxOf<split_t> {
    typedef bf16_t type;
};
template <typename T> using Aux = typename AuxOf<T>::type;

__device__ __forceinline__ void split2(float v, float &hi, float &lo) {
    hi = to_f32(from_f32<bf16_t>(v));
    lo = (__float_as_uint(hi) & 0x7f800000u) == 0x7f800000u ? 0.0f : v - hi;  // exact
}

// One aligned group of 4 values as its 16-byte split piece.
__device__ __forceinline__ u32x4 pack_split4(const float *v) {
    float h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) split2(v[j], h[j], l[j]);
    return u32x4{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3]), pack_bf16x2(l[0], l[1]),
                 pack_bf16x2(l[2], l[3])};
}

template <int V> __device__ __forceinline__ void store_frag(split_t *p, const float (&v)[V]) {
    static_assert(V % 4 == 0, "split stores cover whole groups of 4 elements");
#pragma unroll
    for (int i = 0; i < V / 4; ++i) store_raw(p + 4 * i, pack_split4(v + 4 * i));
}
__device__ __forceinline__ void store_chunk(split_t *p, const float (&v)[4]) {
    store_raw(p, pack_split4(v));
}

// One element at element index e of an output (the general kernels' store).
__device__ __forceinline__ void put_elem(float *p, int64_t e, float v) { p[e] = v; }
__device__ __forceinline__ void put_elem(bf16_t *p, int64_t e, float v) {
    p[e] = from_f32<bf16_t>(v);
}
__device__ __forceinline__ void put_elem(split_t *p, int64_t e, float v) {
    float hi, lo;
    split2(v, hi, lo);
    bf16_t *b = reinterpret_cast<bf16_t *>(p) + 8 * (e >> 2) + (e & 3);
    b[0] = from_f32<bf16_t>(hi);
    b[4] = from_f32<bf16_t>(lo);
}

// ------------------------------------------------------------- reductions --
// Sum over aligned groups of N lanes (N a power of two <= 64) of a wavefront;
// every lane of a group ends with the bit-identical sum (each step adds a pair
// of partial sums that the partner lane adds in the other order, and fp32
// addition is commutative).  Steps inside a 16-lane row use DPP lane swizzles
// (quad permutes, then the half-row and row mirrors, which pair each lane with
// one in the other quad / half).  The 16- and 32-lane steps cross rows with the
// gfx950 lane swaps: permlane16_swap(v, v) returns {v with each odd row replaced
// by the even row before it, v with each even row replaced by the odd row after
// it}, so the two halves sum to v[l] + v[l ^ 16] in the same operand order on
// both partner lanes (permlane32_swap likewise for l ^ 32).
template <int CTRL> __device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float swap_sum16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap_sum32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int N> __device__ __forceinline__ float group_sum(float v) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "group of 1..64 lanes");
    if constexpr (N >= 2) v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (N >= 4) v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
    if constexpr (N >= 8) v += dpp<0x141>(v);  // row_half_mirror: lane 7-i of 8
    if constexpr (N >= 16) v += dpp<0x140>(v); // row_mirror: lane 15-i of 16
    if constexpr (N >= 32) v = swap_sum16(v);  // lane ^ 16
    if constexpr (N >= 64) v = swap_sum32(v);  // lane ^ 32
    return v;
}

// 1 / sqrt(x) as two correctly rounded operations, RN(1 / RN(sqrt(x))): the
// value of 1.0f / sqrtf(x).  For 2^-96 <= x < inf it is built from the hardware
// estimates: v_sqrt_f32's root r is within one ulp, and the residuals
// x - (r -/+ ulp) * r, exact with FMA, pick the rounded root among r - ulp, r and
// r + ulp (the correction LLVM's AMDGPU lowering applies to its f32 square
// root); v_rcp_f32's reciprocal q of that root is refined by one Newton step
// with FMA, q + q * (1 - y * q) (Markstein).  About 12 instructions instead of
// the ~30 of the general sequences, which rescale small inputs and handle
// division overflow.  Equal bit for bit to the general expression for every
// float in that range on MI355X (qdc_row_scale_check sweeps all 2^32 bit
// patterns); other inputs (zero, tiny, inf, NaN, negative) take the general
// expression itself.
__device__ __forceinline__ float inv_sqrt_rn(float x) {
    if (!(x >= 0x1p-96f && x < __builtin_inff())) return 1.0f / __builtin_sqrtf(x);
    const float r = __builtin_amdgcn_sqrtf(x);
    const float dn = __uint_as_float(__float_as_uint(r) - 1u);
    const float up = __uint_as_float(__float_as_uint(r) + 1u);
    float y = r;
    if (__builtin_fmaf(-dn, r, x) <= 0.0f) y = dn;
    if (__builtin_fmaf(-up, r, x) > 0.0f) y = up;
    const float q = __builtin_amdgcn_rcpf(y);
    return __builtin_fmaf(__builtin_fmaf(-y, q, 1.0f), q, q);
}

// 1/sqrt(sum/width + eps) in fp32, the reference's operation order
// (src/backbone_cpu.jl:344): divide, add, square root, reciprocal.  For a
// power-of-two width (uniform: a kernel argument) the division is a multiply by
// the exact reciprocal 2^-k, the same correctly rounded quotient without the
// division sequence; the square root and reciprocal are inv_sqrt_rn.
__device__ __forceinline__ float rms_scale(float sum_squares, float width, float eps) {
    const uint32_t wb = __float_as_uint(width);
    const uint32_t e = wb & 0x7f800000u;
    float mean;
    if ((wb & 0x807fffffu) == 0u && e >= 0x3f800000u && e <= 0x7e800000u)  // 2^k, 0 <= k <= 126
        mean = sum_squares * __uint_as_float(0x7f000000u - e);
    else
        mean = sum_squares / width;
    return inv_sqrt_rn(mean + eps);
}

// silu(x) = x * (1/(1 + exp(-x))) (src/backbone.jl:196-197).  exp(-x) is
// computed as exp2(-x*log2(e)) on the hardware transcendental unit and the
// reciprocal with v_rcp_f32: both within ~1 ulp, ample for the 1e-5 relative
// bar.  Overflow of exp for x < -88 gives 1/inf = 0 and x*0 = -0, as on the CPU.
__device__ __forceinline__ float silu(float x) {
    const float e = __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// ------------------------------------------------------ integer division --
// Division of n < 2^31 by a fixed divisor d >= 1 with one multiply-high, add
// and shift (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, sec. 4): l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1,  q = (mulhi(n, m) + n) >> l.
struct FastDiv {
    uint32_t d, m, l;
};

static inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    const uint64_t m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
    return FastDiv{d, (uint32_t)m, l};
}

__host__ __device__ __forceinline__ uint32_t fastdiv(uint32_t n, const FastDiv &f) {
#ifdef __HIP_DEVICE_COMPILE__
    return (__umulhi(n, f.m) + n) >> f.l;
#else
    return (uint32_t)((((uint64_t)n * f.m) >> 32) + n) >> f.l;
#endif
}

// Internal dispatch result: no fast-path kernel fits the shape.
constexpr int32_t kNoFastPath = INT32_MIN;

// --------------------------------------------------------- host helpers ---
static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }
// Bytes per element; a QDC_BF16X2 element is two bf16 terms.
static inline int64_t elem_size(int32_t dtype) { return dtype == QDC_BF16 ? 2 : 4; }
static inline bool valid_dtype(int32_t dtype) { return dtype == QDC_F32 || dtype == QDC_BF16; }
// A split output's rows must start on a group of 4 elements and hold whole groups.
static inline bool split_rows_ok(int64_t width, int64_t row_stride) {
    return width % 4 == 0 && row_stride % 4 == 0;
}

// Launch status: a positive hipError_t when the launch failed, else 0.
static inline int32_t launch_status() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? QDC_OK : (int32_t)e;
}

static inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Byte ranges [a, a+na) and [b, b+nb) intersect.
static inline bool overlaps(const void *a, int64_t na, const void *b, int64_t nb) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return na > 0 && nb > 0 && x < y + (uintptr_t)nb && y < x + (uintptr_t)na;
}

}  // namespace qdc
