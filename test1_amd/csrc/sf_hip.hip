// Device side of the layer-streaming path for MI355X (gfx950).
//
// Every kernel here is a streaming kernel: each byte is read once and
// written once, so the bound is HBM bandwidth (or the host link, for the
// copies), never the matrix cores.  The kernels therefore use
//   - 128-bit global loads and stores, 8 elements per lane per group,
//   - several independent groups per lane to keep enough bytes in flight,
//   - 128- or 256-lane workgroups (2 or 4 wave64s) and an exact grid of
//     many thousands of workgroups so all 256 CUs over the 8 XCDs stay busy,
//   - no LDS and no MFMA.
//
// The C ABI is declared in include/slidefsdp.h.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
#include <stdint.h>
#include <string.h>

#include <chrono>
#include <mutex>
#include <thread>
#include <unordered_map>

#include "../../include/slidefsdp.h"

namespace {

constexpr int kThreads = 256;  // lanes per workgroup (4 wave64s)
constexpr int kUnroll = 4;     // 8-element groups per lane per workgroup tile
constexpr int kCastUnroll = 1; // the same for the flat cast (measured best, see below)
constexpr int kCastThreads = 128;  // lanes per workgroup of the flat cast (2 wave64s, see below)
constexpr int kGroup = 8;      // elements per 128-bit bf16 store
constexpr uint64_t kTileElems = uint64_t(kThreads) * kUnroll * kGroup;  // 8192

// Native vector types: the nontemporal builtins need them (HIP's float4 is a
// struct), and they map one-to-one onto 128-bit global_load/store_dwordx4.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// fp32 -> bf16 with round-to-nearest-even on the bit pattern, NaN -> 0xFFFF.
// This is the arithmetic of torch's vectorised CPU cast that the reference
// calls at layer_state.py:301 (ATen cvtfp32_bf16: bias 0x7FFF plus the lsb
// of the kept half, and an all-ones pattern for unordered inputs); the
// tests pin it against that routine.  Denormals, infinities and signed
// zeros follow from the integer arithmetic.
__device__ __forceinline__ uint32_t rne_bf16(uint32_t u) {
    const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    return ((u & 0x7FFFFFFFu) > 0x7F800000u) ? 0xFFFFu : r;
}

// fp32 -> fp16, IEEE round to nearest even with subnormals; overflow to
// infinity; NaN -> quiet NaN keeping the sign and the top 9 payload bits.
// This is what torch's CPU cast gives (`.to(torch.float16)`, the reference's
// staging of fp16 units, layer_state.py:301); the tests pin it against that
// routine.  Integer arithmetic only, so the result does not depend on the
// shader's floating-point modes.
__device__ __forceinline__ uint32_t rne_f16(uint32_t u) {
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7E00u | ((a >> 13) & 0x1FFu);   // NaN
    if (a >= 0x477FF000u) return sign | 0x7C00u;                          // rounds past 65504
    if (a >= 0x38800000u) {                                               // normal half
        const uint32_t r = a - 0x38000000u;                               // exponent rebias 127 -> 15
        return sign | ((r + 0xFFFu + ((r >> 13) & 1u)) >> 13);
    }
    const uint32_t e = a >> 23;                                           // subnormal half or zero
    if (e < 102u) return sign;                                            // below half the smallest subnormal
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t s = 126u - e;                                          // 14 .. 24
    const uint32_t q = m >> s, rem = m & ((1u << s) - 1u), half = 1u << (s - 1u);
    return sign | (q + ((rem > half) | ((rem == half) & (q & 1u))));
}

__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) {
    return lo | (hi << 16);
}

__device__ __forceinline__ u32x4 cast8(const f32x4 a, const f32x4 b) {
    u32x4 o;
    o.x = pack2(rne_bf16(__float_as_uint(a.x)), rne_bf16(__float_as_uint(a.y)));
    o.y = pack2(rne_bf16(__float_as_uint(a.z)), rne_bf16(__float_as_uint(a.w)));
    o.z = pack2(rne_bf16(__float_as_uint(b.x)), rne_bf16(__float_as_uint(b.y)));
    o.w = pack2(rne_bf16(__float_as_uint(b.z)), rne_bf16(__float_as_uint(b.w)));
    return o;
}

__device__ __forceinline__ u32x4 cast8_f16(const f32x4 a, const f32x4 b) {
    u32x4 o;
    o.x = pack2(rne_f16(__float_as_uint(a.x)), rne_f16(__float_as_uint(a.y)));
    o.y = pack2(rne_f16(__float_as_uint(a.z)), rne_f16(__float_as_uint(a.w)));
    o.z = pack2(rne_f16(__float_as_uint(b.x)), rne_f16(__float_as_uint(b.y)));
    o.w = pack2(rne_f16(__float_as_uint(b.z)), rne_f16(__float_as_uint(b.w)));
    return o;
}

// Output formats of the flat cast.
struct ToBf16 {
    __device__ static u32x4 cast8(const f32x4 a, const f32x4 b) { return ::cast8(a, b); }
    __device__ static uint16_t cast1(float x) { return uint16_t(rne_bf16(__float_as_uint(x))); }
};
struct ToF16 {
    __device__ static u32x4 cast8(const f32x4 a, const f32x4 b) { return cast8_f16(a, b); }
    __device__ static uint16_t cast1(float x) { return uint16_t(rne_f16(__float_as_uint(x))); }
};

// ---------------------------------------------------------------------
// Flat cast: n8 groups of 8 elements, both pointers 16-byte aligned.
// Workgroup b owns groups [b*kCastThreads*kCastUnroll, (b+1)*kCastThreads*kCastUnroll);
// within it, unroll step k covers one contiguous run of kCastThreads groups,
// so every load/store instruction of a wave touches one contiguous 2 KiB
// span.  Loads and stores are nontemporal 128-bit accesses.  With cached
// loads the cast's rate depended on the work before it, falling with the
// bytes that work had written; with nontemporal loads it does not (one
// Llama layer, 10 casts per case, two rounds on one box, fraction of HBM
// peak):
//                         cached loads   nontemporal loads
//   back to back          0.759-0.763    0.777-0.780
//   after 20 bf16 GEMMs   0.733-0.738    0.766-0.768
//   after 4 x 1 GiB copy  0.676-0.680    0.767-0.769
// The sc0/sc1 bits changed nothing beside nt; plain stores were slower.
// Other shapes, one box each: 2 groups per lane 6.16 TB/s (then with
// nontemporal loads 5.61), 4 groups 6.04, 8 groups 5.70; one group per
// lane, measured in the training step: 0.2172-0.2182 ms per layer alone
// against 0.2245-0.2253 with 2 groups.  Workgroup size, one group per lane,
// two rounds on one box: 64 lanes 0.214 ms, 128 lanes 0.2124-0.2131 (6.15
// TB/s, 0.77 of peak), 256 lanes 0.2144-0.2157, 512 0.216-0.217, 1024
// 0.221-0.222; a plain fp32 copy of the same bytes reaches 0.79 of peak.
// Loads with every lane's 16 bytes contiguous across the wave (then 8-byte
// stores, or 16-byte stores after a lane-pair exchange), a blockIdx order
// that gives each XCD one contiguous eighth, and persistent grid-stride
// loops were no faster.
// ---------------------------------------------------------------------
template <typename Fmt>
__device__ __forceinline__ void cast_flat_body(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                               uint64_t n8) {
    // Highest issue priority among the waves of its SIMD: staged units are
    // cast while the backward's GEMMs run on the same CUs, and the cast's few
    // instructions per byte then issue without queueing behind MFMA waves
    // (in a training step: 0.2537 -> 0.2492 ms per Llama layer).
    __builtin_amdgcn_s_setprio(3);
    const uint64_t tile0 = uint64_t(blockIdx.x) * (kCastThreads * kCastUnroll);
    if (tile0 + kCastThreads * kCastUnroll <= n8) {
        // Full tile (every workgroup but possibly the last): all loads are
        // issued before the first conversion, with no per-lane predicate
        // between them.
        f32x4 a[kCastUnroll], b[kCastUnroll];
#pragma unroll
        for (int k = 0; k < kCastUnroll; ++k) {
            const f32x4* p = reinterpret_cast<const f32x4*>(src + (tile0 + k * kCastThreads + threadIdx.x) * kGroup);
            a[k] = __builtin_nontemporal_load(p);
            b[k] = __builtin_nontemporal_load(p + 1);
        }
#pragma unroll
        for (int k = 0; k < kCastUnroll; ++k) {
            __builtin_nontemporal_store(Fmt::cast8(a[k], b[k]),
                reinterpret_cast<u32x4*>(dst + (tile0 + k * kCastThreads + threadIdx.x) * kGroup));
        }
    } else {
        for (int k = 0; k < kCastUnroll; ++k) {
            const uint64_t g = tile0 + k * kCastThreads + threadIdx.x;
            if (g < n8) {
                const f32x4* p = reinterpret_cast<const f32x4*>(src + g * kGroup);
                __builtin_nontemporal_store(Fmt::cast8(__builtin_nontemporal_load(p), __builtin_nontemporal_load(p + 1)),
                                            reinterpret_cast<u32x4*>(dst + g * kGroup));
            }
        }
    }
}

// The staging cast to bf16 (the default unit dtype) and to fp16.
__global__ __launch_bounds__(kCastThreads) void cast_flat_kernel(
    const float* __restrict__ src, uint16_t* __restrict__ dst, uint64_t n8) {
    cast_flat_body<ToBf16>(src, dst, n8);
}

__global__ __launch_bounds__(kCastThreads) void cast_flat_f16_kernel(
    const float* __restrict__ src, uint16_t* __restrict__ dst, uint64_t n8) {
    cast_flat_body<ToF16>(src, dst, n8);
}

// ---------------------------------------------------------------------
// Row gather: dst row t = src row ids[t] (rows of row_len elements), cast
// fp32 -> bf16 (kCast) or copied as 16-bit values.  One workgroup per row
// per iteration, grid-stride over the rows; src may be pinned host memory
// (the row-sparse embedding load) and dst may be pinned host memory (the
// row-sparse gradient offload, then with a capped grid).  An id outside
// [0, nrows) yields a row of 0xFFFF (a NaN in bf16) and sets *bad.
//
// Each lane issues the loads of kRows 8-element groups of its row (kRows =
// whole groups per lane, 1 to 4, picked at launch from the row length) before
// the first store, so a row crosses the host link in one round trip.  Those
// passes carry no per-lane predicate: under one, the compiler waits for all
// outstanding memory operations before each store, and since stores count as
// outstanding, each store into host memory would wait for the previous one
// to be acknowledged over the link.  The groups left over (fewer than
// kThreads * kRows) go one per lane with a predicate.  With a capped
// 8-workgroup grid for the gradient-row offload (HBM -> pinned host, rows of
// 4096 bf16) the unpredicated two-group pass measured 52.1-53.7 GB/s alone
// against 47.7-48.3 GB/s with one group in flight per lane or with
// predicated stores, and 55.6 GB/s with the offload's 16 workgroups; the
// lookup (host -> HBM, one workgroup per row) is at the link's rate either
// way (53.9 GB/s).
// ---------------------------------------------------------------------
template <bool kCast>
__device__ __forceinline__ u32x4 gather_group(const void* __restrict__ src, uint64_t base, uint64_t g) {
    if (kCast) {
        const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + base + g * kGroup);
        return cast8(p[0], p[1]);
    }
    return reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(src) + base)[g];
}

template <bool kCast, int kRows>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(
    const void* __restrict__ src, const int64_t* __restrict__ ids, uint64_t ntok, uint64_t row_len,
    uint64_t nrows, uint16_t* __restrict__ dst, uint32_t* __restrict__ bad, int vec) {
    for (uint64_t t = blockIdx.x; t < ntok; t += gridDim.x) {
        const int64_t r = ids[t];
        uint16_t* out = dst + t * row_len;
        if (r < 0 || uint64_t(r) >= nrows) {
            for (uint64_t j = threadIdx.x; j < row_len; j += kThreads) out[j] = 0xFFFFu;
            if (bad != nullptr && threadIdx.x == 0) bad[0] = 1u;
            continue;
        }
        const uint64_t base = uint64_t(r) * row_len;
        if (vec) {
            constexpr uint64_t kPass = uint64_t(kThreads) * kRows;
            const uint64_t g8 = row_len / kGroup;
            const uint64_t full = g8 / kPass * kPass;
            for (uint64_t g0 = 0; g0 < full; g0 += kPass) {
                f32x4 a[kRows], b[kRows];
                u32x4 v[kRows];
#pragma unroll
                for (int k = 0; k < kRows; ++k) {
                    const uint64_t g = g0 + uint64_t(k) * kThreads + threadIdx.x;
                    if (kCast) {
                        const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + base +
                                                                       g * kGroup);
                        a[k] = p[0];
                        b[k] = p[1];
                    } else {
                        v[k] = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(src) + base)[g];
                    }
                }
#pragma unroll
                for (int k = 0; k < kRows; ++k) {
                    const uint64_t g = g0 + uint64_t(k) * kThreads + threadIdx.x;
                    __builtin_nontemporal_store(kCast ? cast8(a[k], b[k]) : v[k], reinterpret_cast<u32x4*>(out) + g);
                }
            }
            for (uint64_t g = full + threadIdx.x; g < g8; g += kThreads)
                __builtin_nontemporal_store(gather_group<kCast>(src, base, g), reinterpret_cast<u32x4*>(out) + g);
        } else {
            for (uint64_t j = threadIdx.x; j < row_len; j += kThreads) {
                out[j] = kCast ? uint16_t(rne_bf16(__float_as_uint(static_cast<const float*>(src)[base + j])))
                               : static_cast<const uint16_t*>(src)[base + j];
            }
        }
    }
}

// Scalar cast for tails and for pointers that are not 16-byte aligned.
template <typename Fmt>
__global__ __launch_bounds__(kThreads) void cast_scalar_kernel(
    const float* __restrict__ src, uint16_t* __restrict__ dst, uint64_t n) {
    const uint64_t stride = uint64_t(gridDim.x) * kThreads;
    for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
        dst[i] = Fmt::cast1(src[i]);
    }
}

__global__ __launch_bounds__(kThreads) void fill_b16_kernel(
    uint16_t* __restrict__ dst, uint64_t n, uint16_t value) {
    const uint32_t v2 = uint32_t(value) | (uint32_t(value) << 16);
    const u32x4 v = {v2, v2, v2, v2};
    const uint64_t n8 = n / kGroup;
    const uint64_t base = uint64_t(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x;
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        const uint64_t g = base + uint64_t(k) * kThreads;
        if (g < n8) reinterpret_cast<u32x4*>(dst)[g] = v;
    }
    // tail (< 8 elements): the first lanes of the first workgroup
    if (blockIdx.x == 0 && threadIdx.x < (n - n8 * kGroup)) dst[n8 * kGroup + threadIdx.x] = value;
}

// ---------------------------------------------------------------------
// Segment-table kernels.  The table travels in the kernel arguments
// (about 2 KiB for SF_MAX_SEGS segments), so no device allocation is
// needed.  Each workgroup owns one tile of kTileElems elements inside a
// single segment: tiles are numbered across segments and tile_start[s]
// is the first tile of segment s.  A workgroup finds its segment with a
// binary search over tile_start, whose loads are uniform (scalar).
// ---------------------------------------------------------------------
struct SegTable {
    uint64_t src[SF_MAX_SEGS];
    uint64_t dst[SF_MAX_SEGS];
    uint64_t n[SF_MAX_SEGS];
    uint64_t tile_start[SF_MAX_SEGS + 1];
    uint32_t nsegs;
};

__device__ __forceinline__ uint32_t find_seg(const SegTable& t, uint64_t tile) {
    uint32_t lo = 0, hi = t.nsegs;  // tile_start[lo] <= tile < tile_start[hi]
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (t.tile_start[mid] <= tile) lo = mid; else hi = mid;
    }
    return lo;
}

// Element operations: fp32 -> bf16 cast, or 16-bit copy.
struct OpCast {
    using S = float;
    __device__ static u32x4 load_convert(const S* p) {
        const f32x4* q = reinterpret_cast<const f32x4*>(p);
        return cast8(__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1));
    }
    __device__ static uint16_t convert1(S x) { return uint16_t(rne_bf16(__float_as_uint(x))); }
    static constexpr uint64_t kAlign = 16;  // both sides need 16-byte alignment
};

struct OpCopy16 {
    using S = uint16_t;
    __device__ static u32x4 load_convert(const S* p) {
        return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    }
    __device__ static uint16_t convert1(S x) { return x; }
    static constexpr uint64_t kAlign = 16;
};

template <typename Op>
__global__ __launch_bounds__(kThreads) void seg_kernel(const SegTable t) {
    using S = typename Op::S;
    const uint64_t ntiles = t.tile_start[t.nsegs];
    // Grid-stride over tiles: one workgroup per tile when the grid covers
    // them all, or a capped grid (e.g. a copy into host memory, which only
    // needs enough workgroups to keep the host link busy).
    for (uint64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const uint32_t s = find_seg(t, tile);
        const uint64_t first = (tile - t.tile_start[s]) * kTileElems;  // element offset in segment
        const uint64_t n = t.n[s];
        const uint64_t len = (n - first < kTileElems) ? (n - first) : kTileElems;
        const S* src = reinterpret_cast<const S*>(t.src[s]) + first;
        uint16_t* dst = reinterpret_cast<uint16_t*>(t.dst[s]) + first;

        const bool aligned = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) &
                              (Op::kAlign - 1)) == 0;
        if (aligned && len == kTileElems) {
            // Full aligned tile: unpredicated loads, all in flight together.
            u32x4 v[kUnroll];
#pragma unroll
            for (int k = 0; k < kUnroll; ++k) v[k] = Op::load_convert(src + (k * kThreads + threadIdx.x) * kGroup);
#pragma unroll
            for (int k = 0; k < kUnroll; ++k)
                __builtin_nontemporal_store(v[k], reinterpret_cast<u32x4*>(dst + (k * kThreads + threadIdx.x) * kGroup));
        } else if (aligned) {
            // Last tile of a segment: predicated groups, then the < 8 element tail.
            const uint64_t n8 = len / kGroup;
            for (int k = 0; k < kUnroll; ++k) {
                const uint64_t g = k * kThreads + threadIdx.x;
                if (g < n8) __builtin_nontemporal_store(Op::load_convert(src + g * kGroup),
                                                        reinterpret_cast<u32x4*>(dst + g * kGroup));
            }
            const uint64_t rem = len - n8 * kGroup;
            if (threadIdx.x < rem) dst[n8 * kGroup + threadIdx.x] = Op::convert1(src[n8 * kGroup + threadIdx.x]);
        } else {
            for (uint64_t i = threadIdx.x; i < len; i += kThreads) dst[i] = Op::convert1(src[i]);
        }
    }
}

inline uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// Upper bound on workgroups per launch; the grids below stay far under the
// 2^32-1 lanes per dimension that the dispatch packet allows.
constexpr uint64_t kMaxBlocks = (uint64_t(1) << 31) / kThreads;

template <typename Op>
int launch_segs(const sf_seg* segs, int nsegs, int max_workgroups, hipStream_t stream) {
    if (nsegs < 0 || (nsegs > 0 && segs == nullptr)) return SF_EINVAL;
    // Tables longer than SF_MAX_SEGS are split into several launches.
    for (int base = 0; base < nsegs; base += SF_MAX_SEGS) {
        const int cnt = (nsegs - base < SF_MAX_SEGS) ? (nsegs - base) : SF_MAX_SEGS;
        SegTable t;
        memset(&t, 0, sizeof(t));
        uint64_t tiles = 0;
        uint32_t m = 0;
        for (int i = 0; i < cnt; ++i) {
            const sf_seg& g = segs[base + i];
            if (g.n == 0) continue;
            if (g.src == 0 || g.dst == 0) return SF_EINVAL;
            t.src[m] = g.src;
            t.dst[m] = g.dst;
            t.n[m] = g.n;
            t.tile_start[m] = tiles;
            tiles += ceil_div(g.n, kTileElems);
            ++m;
        }
        if (m == 0) continue;
        t.tile_start[m] = tiles;
        t.nsegs = m;
        if (tiles > kMaxBlocks) return SF_EINVAL;  // > 17.6e12 elements: not a real layer
        uint64_t grid = tiles;
        if (max_workgroups > 0 && grid > uint64_t(max_workgroups)) grid = uint64_t(max_workgroups);
        hipLaunchKernelGGL(seg_kernel<Op>, dim3(uint32_t(grid)), dim3(kThreads), 0, stream, t);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return int(e);
    }
    return SF_OK;
}

}  // namespace

namespace {
// Status of a failed runtime call, handed to the caller.  The runtime also
// keeps it as the thread's last error, where the next library that checks
// for errors (torch after its own calls) would report it as its own: clear it.
inline int hip_status(hipError_t e) {
    if (e != hipSuccess) (void)hipGetLastError();
    return int(e);
}
}  // namespace

namespace {
template <bool kCast>
int launch_gather_rows(const void* src, const int64_t* ids, size_t ntok, size_t row_len, size_t nrows,
                       uint16_t* dst, uint32_t* bad, int max_workgroups, hipStream_t st, size_t src_elem) {
    if (ntok == 0 || row_len == 0) return SF_OK;
    if (src == nullptr || ids == nullptr || dst == nullptr) return SF_EINVAL;
    if ((reinterpret_cast<uintptr_t>(dst) & 1) != 0) return SF_EINVAL;
    // the destination rows must not overlap the source table
    const uintptr_t s0 = reinterpret_cast<uintptr_t>(src), d0 = reinterpret_cast<uintptr_t>(dst);
    if (s0 < d0 + 2 * ntok * row_len && d0 < s0 + src_elem * nrows * row_len) return SF_EOVERLAP;
    const int vec = (row_len % kGroup == 0) && ((s0 | d0) & 15) == 0;
    uint64_t grid = ntok;
    if (max_workgroups > 0 && grid > uint64_t(max_workgroups)) grid = uint64_t(max_workgroups);
    if (grid > kMaxBlocks) grid = kMaxBlocks;
    // whole groups of 8 per lane and pass, 1 to 4
    const uint64_t per_lane = (row_len / kGroup) / kThreads;
    auto kernel = per_lane >= 4 ? gather_rows_kernel<kCast, 4>
                : per_lane == 3 ? gather_rows_kernel<kCast, 3>
                : per_lane == 2 ? gather_rows_kernel<kCast, 2>
                                : gather_rows_kernel<kCast, 1>;
    hipLaunchKernelGGL(kernel, dim3(uint32_t(grid)), dim3(kThreads), 0, st, src, ids, uint64_t(ntok),
                       uint64_t(row_len), uint64_t(nrows), dst, bad, vec);
    return hip_status(hipGetLastError());
}
}  // namespace

extern "C" {

const char* sf_error_string(int status) {
    switch (status) {
        case SF_OK: return "success";
        case SF_EINVAL: return "sf: invalid argument (null pointer, bad size or enum)";
        case SF_ETOOMANY: return "sf: too many segments for one call";
        case SF_EDTYPE: return "sf: dtype combination not supported";
        case SF_ENOOPT: return "sf: unknown optimizer id";
        case SF_EOVERLAP: return "sf: source and destination overlap";
        case SF_ETOOBIG: return "sf: piece larger than the library's device scratch (SF_STAGE_SCRATCH_ELEMS)";
        case SF_ETIMEDOUT: return "sf: wait ended at its deadline with work still pending";
        default:
            if (status >= SF_EDMA_BASE && status < SF_EDMA_BASE + 0x1000) return "sf: ROCr DMA call failed";
            return hipGetErrorString(hipError_t(status));
    }
}

int sf_abi_version(void) { return SF_ABI_VERSION; }

}  // extern "C"

namespace {

// The flat cast's launches: the vector kernel over the 8-element groups (when
// both pointers are 16-byte aligned), then the scalar kernel over the rest.
// ``start`` / ``stop`` (may be null) are stamped by the runtime around the
// first and the last launch's own dispatch, so they time the kernels alone,
// not what the stream waited for before them.
int cast_launch(const float* src, uint16_t* dst, size_t n, hipStream_t st, hipEvent_t start, hipEvent_t stop,
                bool to_f16 = false) {
    if (n == 0) {
        // nothing to launch: the events still mark the (empty) interval
        if (start != nullptr) {
            const hipError_t e = hipEventRecord(start, st);
            if (e != hipSuccess) return hip_status(e);
        }
        if (stop != nullptr) {
            const hipError_t e = hipEventRecord(stop, st);
            if (e != hipSuccess) return hip_status(e);
        }
        return SF_OK;
    }
    if (src == nullptr || dst == nullptr) return SF_EINVAL;
    const uintptr_t s = reinterpret_cast<uintptr_t>(src), d = reinterpret_cast<uintptr_t>(dst);
    // fp32 source [s, s+4n) and bf16 destination [d, d+2n) must not overlap:
    // workgroups run in no particular order.
    if (s < d + 2 * n && d < s + 4 * n) return SF_EOVERLAP;
    const uint64_t n8 = ((s | d) & 15) == 0 ? n / kGroup : 0;
    const uint64_t done = n8 * kGroup;
    const bool tail = done < n;
    if (n8 > 0) {
        const uint64_t blocks = ceil_div(n8, uint64_t(kCastThreads) * kCastUnroll);
        if (blocks > kMaxBlocks) return SF_EINVAL;
        hipExtLaunchKernelGGL(to_f16 ? cast_flat_f16_kernel : cast_flat_kernel, dim3(uint32_t(blocks)),
                              dim3(kCastThreads), 0, st, start, tail ? nullptr : stop, 0, src, dst, n8);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return int(e);
    }
    if (tail) {
        const uint64_t rest = n - done;
        uint64_t blocks = ceil_div(rest, kThreads);
        if (blocks > 65536) blocks = 65536;
        hipExtLaunchKernelGGL(to_f16 ? cast_scalar_kernel<ToF16> : cast_scalar_kernel<ToBf16>, dim3(uint32_t(blocks)),
                              dim3(kThreads), 0, st, n8 > 0 ? nullptr : start, stop, 0, src + done, dst + done, rest);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return int(e);
    }
    return SF_OK;
}

}  // namespace

extern "C" {

int sf_cast_f32_bf16(const float* src, uint16_t* dst, size_t n, sf_stream_t stream) {
    return cast_launch(src, dst, n, reinterpret_cast<hipStream_t>(stream), nullptr, nullptr);
}

int sf_cast_f32_bf16_timed(const float* src, uint16_t* dst, size_t n, sf_stream_t stream, sf_event_t start,
                           sf_event_t stop) {
    if ((start == nullptr) != (stop == nullptr)) return SF_EINVAL;
    return cast_launch(src, dst, n, reinterpret_cast<hipStream_t>(stream), reinterpret_cast<hipEvent_t>(start),
                       reinterpret_cast<hipEvent_t>(stop));
}

int sf_cast_f32_f16(const float* src, uint16_t* dst, size_t n, sf_stream_t stream) {
    return cast_launch(src, dst, n, reinterpret_cast<hipStream_t>(stream), nullptr, nullptr, true);
}

int sf_cast_f32_f16_timed(const float* src, uint16_t* dst, size_t n, sf_stream_t stream, sf_event_t start,
                          sf_event_t stop) {
    if ((start == nullptr) != (stop == nullptr)) return SF_EINVAL;
    return cast_launch(src, dst, n, reinterpret_cast<hipStream_t>(stream), reinterpret_cast<hipEvent_t>(start),
                       reinterpret_cast<hipEvent_t>(stop), true);
}

int sf_event_create(sf_event_t* ev) {
    if (ev == nullptr) return SF_EINVAL;
    hipEvent_t e = nullptr;
    const int rc = hip_status(hipEventCreate(&e));
    *ev = rc == SF_OK ? reinterpret_cast<sf_event_t>(e) : nullptr;
    return rc;
}

int sf_event_destroy(sf_event_t ev) {
    if (ev == nullptr) return SF_OK;
    return hip_status(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
}

int sf_event_elapsed_ms(sf_event_t start, sf_event_t stop, float* ms) {
    if (start == nullptr || stop == nullptr || ms == nullptr) return SF_EINVAL;
    return hip_status(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)));
}

int sf_cast_scatter_f32_bf16(const sf_seg* segs, int nsegs, sf_stream_t stream) {
    return launch_segs<OpCast>(segs, nsegs, 0, reinterpret_cast<hipStream_t>(stream));
}

int sf_copy_segs_b16(const sf_seg* segs, int nsegs, int max_workgroups, sf_stream_t stream) {
    return launch_segs<OpCopy16>(segs, nsegs, max_workgroups, reinterpret_cast<hipStream_t>(stream));
}

int sf_pack_b16(const sf_seg* segs, int nsegs, uint16_t* dst, int max_workgroups, sf_stream_t stream) {
    if (nsegs < 0 || (nsegs > 0 && (segs == nullptr || dst == nullptr))) return SF_EINVAL;
    sf_seg local[SF_MAX_SEGS];
    uint64_t off = 0;
    for (int base = 0; base < nsegs; base += SF_MAX_SEGS) {
        const int cnt = (nsegs - base < SF_MAX_SEGS) ? (nsegs - base) : SF_MAX_SEGS;
        for (int i = 0; i < cnt; ++i) {
            local[i].src = segs[base + i].src;
            local[i].dst = reinterpret_cast<uint64_t>(dst + off);
            local[i].n = segs[base + i].n;
            off += segs[base + i].n;
        }
        int rc = launch_segs<OpCopy16>(local, cnt, max_workgroups, reinterpret_cast<hipStream_t>(stream));
        if (rc != SF_OK) return rc;
    }
    return SF_OK;
}

int sf_unpack_b16(const uint16_t* src, const sf_seg* segs, int nsegs, int max_workgroups,
                  sf_stream_t stream) {
    if (nsegs < 0 || (nsegs > 0 && (segs == nullptr || src == nullptr))) return SF_EINVAL;
    sf_seg local[SF_MAX_SEGS];
    uint64_t off = 0;
    for (int base = 0; base < nsegs; base += SF_MAX_SEGS) {
        const int cnt = (nsegs - base < SF_MAX_SEGS) ? (nsegs - base) : SF_MAX_SEGS;
        for (int i = 0; i < cnt; ++i) {
            local[i].src = reinterpret_cast<uint64_t>(src + off);
            local[i].dst = segs[base + i].dst;
            local[i].n = segs[base + i].n;
            off += segs[base + i].n;
        }
        int rc = launch_segs<OpCopy16>(local, cnt, max_workgroups, reinterpret_cast<hipStream_t>(stream));
        if (rc != SF_OK) return rc;
    }
    return SF_OK;
}

int sf_gather_rows_f32_bf16(const float* src, const int64_t* ids, size_t ntok, size_t row_len, size_t nrows,
                            uint16_t* dst, uint32_t* bad, int max_workgroups, sf_stream_t stream) {
    return launch_gather_rows<true>(src, ids, ntok, row_len, nrows, dst, bad, max_workgroups,
                                    reinterpret_cast<hipStream_t>(stream), 4);
}

int sf_gather_rows_b16(const uint16_t* src, const int64_t* ids, size_t ntok, size_t row_len, size_t nrows,
                       uint16_t* dst, uint32_t* bad, int max_workgroups, sf_stream_t stream) {
    return launch_gather_rows<false>(src, ids, ntok, row_len, nrows, dst, bad, max_workgroups,
                                     reinterpret_cast<hipStream_t>(stream), 2);
}

int sf_fill_b16(uint16_t* dst, size_t n, uint16_t value, sf_stream_t stream) {
    if (n == 0) return SF_OK;
    if (dst == nullptr) return SF_EINVAL;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if ((reinterpret_cast<uintptr_t>(dst) & 1) != 0) return SF_EINVAL;  // not 16-bit aligned
    if ((reinterpret_cast<uintptr_t>(dst) & 15) != 0) {
        // Fill the head up to the next 16-byte boundary (< 8 elements) with a
        // one-workgroup launch whose vector part is empty, then the rest.
        const uint64_t head = (16 - (reinterpret_cast<uintptr_t>(dst) & 15)) / 2;
        const uint64_t h = head < n ? head : n;
        hipLaunchKernelGGL(fill_b16_kernel, dim3(1), dim3(kThreads), 0, st, dst, h, value);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return int(e);
        dst += h;
        n -= h;
        if (n == 0) return SF_OK;
    }
    const uint64_t n8 = n / kGroup;
    uint64_t blocks = ceil_div(n8 > 0 ? n8 : 1, uint64_t(kThreads) * kUnroll);
    if (blocks > kMaxBlocks) return SF_EINVAL;
    hipLaunchKernelGGL(fill_b16_kernel, dim3(uint32_t(blocks)), dim3(kThreads), 0, st, dst, n, value);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? SF_OK : int(e);
}

}  // extern "C"

// ---------------------------------------------------------------------
// Staging: pinned fp32 host array -> bf16 device array, through a device
// fp32 buffer, all on one stream.  Each piece is copied into the buffer by
// DMA and cast from it by cast_flat_kernel; the next piece's copy into the
// same buffer follows that cast in stream order.  With one stream the copy
// and the cast do not overlap; the cast moves 1.5x the copy's bytes over
// HBM at ~100x the host link's rate, so it adds ~1-2 % to the copy.
// ---------------------------------------------------------------------
namespace {

// The memory type the runtime records for ptr, or -1 for memory it does
// not know (pageable host memory).
int memory_type(const void* p) {
    hipPointerAttribute_t a;
    const hipError_t e = hipPointerGetAttributes(&a, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return -1;
    }
    return int(a.type);
}

int stage_launch(const float* host, uint16_t* dst, size_t n, float* buf, size_t chunk, hipStream_t st) {
    if (n == 0) return SF_OK;
    if (host == nullptr || dst == nullptr || buf == nullptr) return SF_EINVAL;
    // an asynchronous copy needs pinned host memory; the cast writes device memory
    if (memory_type(host) != int(hipMemoryTypeHost) || memory_type(dst) != int(hipMemoryTypeDevice))
        return SF_EINVAL;
    chunk -= chunk % kGroup;  // every piece starts 16-byte aligned in dst if dst does
    if (chunk == 0) return SF_EINVAL;
    for (size_t off = 0; off < n; off += chunk) {
        const size_t c = n - off < chunk ? n - off : chunk;
        const hipError_t e = hipMemcpyAsync(buf, host + off, c * sizeof(float), hipMemcpyHostToDevice, st);
        if (e != hipSuccess) return hip_status(e);
        const int rc = cast_launch(buf, dst + off, c, st, nullptr, nullptr);
        if (rc != SF_OK) return rc;
    }
    return SF_OK;
}

}  // namespace

extern "C" {

int sf_stage_f32_bf16(const float* host_src, uint16_t* dst, size_t n, float* workspace, size_t workspace_elems,
                      sf_stream_t stream) {
    if (n > 0 && (workspace == nullptr || memory_type(workspace) != int(hipMemoryTypeDevice))) return SF_EINVAL;
    return stage_launch(host_src, dst, n, workspace, workspace_elems, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"

// ---------------------------------------------------------------------
// Staging without allocating: the pieces go through the library's own
// device buffer instead of a caller workspace.  `scratch` is a static
// device array, so every device the library's code object is loaded on
// holds one for the life of the process.  In host code its name is not a
// device address: the address comes from hipGetSymbolAddress, looked up
// once per device with that device current, and only that address is
// passed to the copies and the cast.
// ---------------------------------------------------------------------
namespace {

__device__ __align__(256) float scratch[SF_STAGE_SCRATCH_ELEMS];

constexpr int kMaxDevices = 64;
// Per device: the address of `scratch`, and an event recorded after the last
// cast of the previous call (the next call's stream waits on it).  The
// mutex is held from the wait to the record, so the calls of several host
// threads are ordered one after the other.
struct ScratchState {
    float* ptr = nullptr;
    hipEvent_t last = nullptr;
    bool recorded = false;
};
std::mutex g_scratch_mu;
ScratchState g_scratch[kMaxDevices];

// The current device, which must be the device of `st` (the null stream:
// the current device), after the one-time set-up of its scratch state.
int scratch_device_for_stream(hipStream_t st, int* dev) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_status(e);
    if (st != nullptr) {
        hipDevice_t sd = 0;
        e = hipStreamGetDevice(st, &sd);
        if (e != hipSuccess) return hip_status(e);
        if (int(sd) != cur) return SF_EINVAL;
    }
    if (cur < 0 || cur >= kMaxDevices) return SF_EINVAL;
    ScratchState& s = g_scratch[cur];
    if (s.ptr == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e);
        if (p == nullptr) return SF_EINVAL;
        if (s.last == nullptr) {
            e = hipEventCreateWithFlags(&s.last, hipEventDisableTiming);
            if (e != hipSuccess) return hip_status(e);
        }
        s.ptr = static_cast<float*>(p);
    }
    *dev = cur;
    return SF_OK;
}

}  // namespace

extern "C" {

int sf_stage_f32_bf16_noalloc(const float* host_src, uint16_t* dst, size_t n, size_t chunk_elems,
                              sf_stream_t stream) {
    if (chunk_elems > SF_STAGE_SCRATCH_ELEMS) return SF_ETOOBIG;
    if (n == 0) return SF_OK;
    if (host_src == nullptr || dst == nullptr) return SF_EINVAL;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    int dev = 0;
    int rc = scratch_device_for_stream(st, &dev);
    if (rc != SF_OK) return rc;
    ScratchState& s = g_scratch[dev];
    if (s.recorded) {
        const hipError_t e = hipStreamWaitEvent(st, s.last, 0);
        if (e != hipSuccess) return hip_status(e);
    }
    rc = stage_launch(host_src, dst, n, s.ptr, chunk_elems == 0 ? SF_STAGE_SCRATCH_ELEMS : chunk_elems, st);
    // Recorded also after a failed launch: whatever was enqueued before the
    // failure still uses the scratch buffer and must precede the next call.
    const hipError_t e = hipEventRecord(s.last, st);
    if (e == hipSuccess) s.recorded = true;
    if (rc != SF_OK) return rc;
    return hip_status(e);
}

int sf_memcpy_async(void* dst, const void* src, size_t bytes, int kind, sf_stream_t stream) {
    if (bytes == 0) return SF_OK;
    if (dst == nullptr || src == nullptr) return SF_EINVAL;
    hipMemcpyKind k;
    switch (kind) {
        case SF_COPY_H2D: k = hipMemcpyHostToDevice; break;
        case SF_COPY_D2H: k = hipMemcpyDeviceToHost; break;
        case SF_COPY_D2D: k = hipMemcpyDeviceToDevice; break;
        default: return SF_EINVAL;
    }
    return hip_status(hipMemcpyAsync(dst, src, bytes, k, reinterpret_cast<hipStream_t>(stream)));
}

int sf_host_alloc(void** out, size_t bytes) {
    if (out == nullptr) return SF_EINVAL;
    *out = nullptr;
    if (bytes == 0) return SF_OK;
    return hip_status(hipHostMalloc(out, bytes, hipHostMallocDefault));
}

int sf_host_free(void* ptr) {
    if (ptr == nullptr) return SF_OK;
    return hip_status(hipHostFree(ptr));
}

int sf_host_device_pointer(void* host_ptr, void** device_ptr) {
    if (host_ptr == nullptr || device_ptr == nullptr) return SF_EINVAL;
    *device_ptr = nullptr;
    return hip_status(hipHostGetDevicePointer(device_ptr, host_ptr, 0));
}

// ---------------------------------------------------------------------
// SDMA copies device -> pinned host, issued through the ROCr runtime.
//
// hipMemcpyAsync performs device-to-host copies with a shader blit kernel;
// a kernel writing over PCIe slows every HBM-bound kernel running beside it
// (the staging cast takes 5-10x longer), wherever its waves are placed.  An
// SDMA engine moves the same bytes at the same link rate without touching
// the shader memory path.  These copies are not ordered with HIP streams:
// the caller makes sure the source is complete (an event synchronised on the
// host) before sf_dma_copy and reads the destination only after sf_dma_wait.
// ---------------------------------------------------------------------
namespace {
struct DmaAgents {
    hsa_agent_t gpu{0};
    hsa_agent_t cpu{0};
    int device = -1;
    bool ok = false;
    uint32_t engine_mask = 0;  // one SDMA engine bit; 0: runtime's choice
    uint64_t ts_freq = 0;      // HSA system timestamp ticks per second
    int avoid_held = 0;        // route around engines another client holds:
                               // 0 no (default), 1 onto free engines 0-3,
                               // 2 also 4 and up
    // Copies issued here and not yet released by sf_dma_wait: signal handle
    // -> engine bit (0 for a runtime-chosen engine).
    std::unordered_map<uint64_t, uint32_t> outstanding;
};
DmaAgents g_dma;
std::mutex g_dma_mu;

struct AgentScan {
    uint32_t want_bdf;
    hsa_agent_t gpu{0};
    hsa_agent_t first_gpu{0};
    hsa_agent_t cpu{0};
};

hsa_status_t scan_agent(hsa_agent_t a, void* data) {
    AgentScan* sc = static_cast<AgentScan*>(data);
    hsa_device_type_t t;
    if (hsa_agent_get_info(a, HSA_AGENT_INFO_DEVICE, &t) != HSA_STATUS_SUCCESS) return HSA_STATUS_SUCCESS;
    if (t == HSA_DEVICE_TYPE_CPU && sc->cpu.handle == 0) sc->cpu = a;
    if (t == HSA_DEVICE_TYPE_GPU) {
        if (sc->first_gpu.handle == 0) sc->first_gpu = a;
        uint32_t bdf = 0;
        if (hsa_agent_get_info(a, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_BDFID), &bdf) ==
                HSA_STATUS_SUCCESS && bdf == sc->want_bdf && sc->gpu.handle == 0)
            sc->gpu = a;
    }
    return HSA_STATUS_SUCCESS;
}

int hsa_status_to_sf(hsa_status_t s) { return s == HSA_STATUS_SUCCESS ? SF_OK : SF_EDMA_BASE + int(s & 0xFFF); }
}  // namespace

// The runtime reports an engine as unavailable while any copy is pending on
// it: ours, or one of HIP's.  A HIP copy ordered after an event that has not
// fired yet sits on its engine until the event fires, and a copy of ours
// queued on that engine waits behind it (measured: 190 ms behind one such
// H2D).  So an engine of the preferred set that is busy while none of our
// copies is pending on it is held by another client: use the free engines
// among the first four in its place.  Engines 4 and up move host copies at a
// fraction of the rate; mode 2 takes them (twice as many) only when no
// engine among the first four can be had (measured in the fp32 Qwen2.5-14B
// step: gradient copies had waited ~300 ms behind held engines, and the host
// AdamW with them).  An engine that holds a copy of ours counts as ours even
// if another client's copy waits behind it; that client's copy then blocks
// only what is queued after it.
uint32_t sf_dma_choose_engines(uint32_t preferred, uint32_t avail, uint32_t ours, int mode) {
    preferred &= 0xFFFFu;
    if (preferred == 0 || mode <= 0) return preferred;
    const uint32_t held = ~avail & ~ours & 0xFFFFu;
    if ((preferred & held) == 0) return preferred;
    uint32_t use = preferred & ~held;
    const int want = __builtin_popcount(preferred);
    for (int e = 0; e < 4 && __builtin_popcount(use) < want; ++e) {
        const uint32_t b = 1u << e;
        if ((avail & b) && !(use & b)) use |= b;
    }
    if (use == 0 && mode >= 2) {
        for (int e = 4; e < 16 && __builtin_popcount(use) < 2 * want; ++e)
            if (avail & (1u << e)) use |= 1u << e;
    }
    return use != 0 ? use : preferred;
}

namespace {
// Engines for the next device -> host copies, from the runtime's engine
// status and this library's pending copies.  Called with g_dma_mu held.
uint32_t pick_engines_locked(uint32_t preferred, hsa_agent_t cpu, hsa_agent_t gpu) {
    if (preferred == 0 || g_dma.avoid_held <= 0) return preferred;
    uint32_t avail = 0;
    if (hsa_amd_memory_copy_engine_status(cpu, gpu, &avail) != HSA_STATUS_SUCCESS) return preferred;
    uint32_t ours = 0;
    for (const auto& kv : g_dma.outstanding)
        if (hsa_signal_load_scacquire(hsa_signal_t{kv.first}) >= 1) ours |= kv.second;
    return sf_dma_choose_engines(preferred, avail, ours, g_dma.avoid_held);
}
}  // namespace

int sf_dma_init(int device) {
    std::lock_guard<std::mutex> lk(g_dma_mu);
    if (g_dma.ok && g_dma.device == device) return SF_OK;
    hsa_status_t st = hsa_init();  // reference-counted; HIP holds its own reference
    if (st != HSA_STATUS_SUCCESS) return hsa_status_to_sf(st);
    // Match the HIP device to its ROCr agent by PCI location.
    int bus = 0, dev = 0, dom = 0;
    hipError_t e = hipDeviceGetAttribute(&bus, hipDeviceAttributePciBusId, device);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&dev, hipDeviceAttributePciDeviceId, device);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&dom, hipDeviceAttributePciDomainID, device);
    if (e != hipSuccess) return int(e);
    AgentScan sc;
    sc.want_bdf = (uint32_t(bus) << 8) | (uint32_t(dev) << 3);  // function 0
    st = hsa_iterate_agents(scan_agent, &sc);
    if (st != HSA_STATUS_SUCCESS) return hsa_status_to_sf(st);
    if (sc.gpu.handle == 0) sc.gpu = sc.first_gpu;  // single-GPU fallback
    if (sc.gpu.handle == 0 || sc.cpu.handle == 0) return SF_EINVAL;
    g_dma.gpu = sc.gpu;
    g_dma.cpu = sc.cpu;
    g_dma.device = device;
    // Copy profiling times come in system timestamp ticks.
    uint64_t freq = 0;
    if (hsa_system_get_info(HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY, &freq) != HSA_STATUS_SUCCESS) freq = 0;
    g_dma.ts_freq = freq;
    g_dma.ok = true;
    // Engine for device -> host copies.  HIP puts each of its own
    // host<->device copies on the first SDMA engine that is free: engine 0,
    // then 1 while 0 is held, then 2.  A HIP copy whose stream waits on an
    // event holds its engine until the event completes, and a copy queued
    // behind it on that engine waits as long (measured on MI355X: with
    // engines 0 and 1 held, a HIP copy waiting for 250 ms of GEMMs took
    // engine 2, and a 1 GiB device -> host copy split over engines 2 and 3
    // took 206 ms instead of 19-21; in the Qwen2.5-14B step the gradient
    // copies on engines 2 and 3 moved 20-28 GB/s while busy, on engine 3
    // alone 52-53).  Engines 0-3 each move 57 GB/s device -> host alone and
    // 52 beside a host -> device copy on another engine, as much as two of
    // them; engines 4-7 move ~25 GB/s together.  So the copies use engine 3
    // alone, the last fast engine HIP reaches, else engine 2, else the
    // runtime's choice.
    // An engine the status reports busy may only be running a copy at this
    // moment: ask again for up to 100 ms before settling for another one.
    g_dma.engine_mask = 0;
    uint32_t seen = 0;
    for (int tries = 0; tries < 100; ++tries) {
        uint32_t avail = 0;
        if (hsa_amd_memory_copy_engine_status(g_dma.cpu, g_dma.gpu, &avail) != HSA_STATUS_SUCCESS) break;
        seen |= avail;
        if (seen & (1u << 3)) break;
        std::this_thread::sleep_for(std::chrono::milliseconds(1));
    }
    if (seen & (1u << 3))
        g_dma.engine_mask = 1u << 3;
    else if (seen & (1u << 2))
        g_dma.engine_mask = 1u << 2;
    return SF_OK;
}

int sf_dma_set_engines(uint32_t engine_mask) {
    std::lock_guard<std::mutex> lk(g_dma_mu);
    if (!g_dma.ok) return SF_EINVAL;
    g_dma.engine_mask = engine_mask & 0xFFFFu;
    return SF_OK;
}

int sf_dma_set_avoid_held(int mode) {
    std::lock_guard<std::mutex> lk(g_dma_mu);
    if (!g_dma.ok) return SF_EINVAL;
    if (mode < 0 || mode > 2) return SF_EINVAL;
    g_dma.avoid_held = mode;
    return SF_OK;
}

int sf_dma_get_engines(uint32_t* engine_mask) {
    std::lock_guard<std::mutex> lk(g_dma_mu);
    if (!g_dma.ok || engine_mask == nullptr) return SF_EINVAL;
    *engine_mask = g_dma.engine_mask;
    return SF_OK;
}

// On an error after some copies were issued, *nsignals holds their number and
// signals[0 .. *nsignals) their handles: those copies run to completion, and
// the caller waits for them (sf_dma_wait) before reusing the destination.
int sf_dma_copy_d2h(const sf_seg* segs, int nsegs, uint64_t* signals, int max_signals, int* nsignals) {
    if (nsegs < 0 || (nsegs > 0 && (segs == nullptr || signals == nullptr)) || nsignals == nullptr) return SF_EINVAL;
    *nsignals = 0;
    uint32_t mask = 0;
    hsa_agent_t cpu{0}, gpu{0};
    {
        std::lock_guard<std::mutex> lk(g_dma_mu);
        if (!g_dma.ok) return SF_EINVAL;
        // Every segment is checked before the first copy is issued.
        for (int i = 0; i < nsegs; ++i)
            if (segs[i].n != 0 && (segs[i].src == 0 || segs[i].dst == 0)) return SF_EINVAL;
        cpu = g_dma.cpu;
        gpu = g_dma.gpu;
        mask = pick_engines_locked(g_dma.engine_mask, cpu, gpu);
    }
    // Engines to spread over: the set bits of the engine mask, or one
    // runtime-chosen engine.
    uint32_t engines[16];
    int nengines = 0;
    for (int e = 0; e < 16; ++e)
        if (mask & (1u << e)) engines[nengines++] = 1u << e;
    if (nengines == 0) engines[nengines++] = 0;
    constexpr uint64_t kSplit = uint64_t(4) << 20;  // split copies above 4 MiB
    int rr = 0;
    for (int i = 0; i < nsegs; ++i) {
        const uint64_t bytes = segs[i].n;
        if (bytes == 0) continue;
        const int parts = (bytes >= kSplit && nengines > 1) ? nengines : 1;
        const uint64_t chunk = (bytes / parts) & ~uint64_t(4095);
        for (int k = 0; k < parts; ++k) {
            const uint64_t off = chunk * k;
            const uint64_t n = (k == parts - 1) ? bytes - off : chunk;
            if (*nsignals >= max_signals) return SF_ETOOMANY;
            hsa_signal_t sig;
            hsa_status_t st = hsa_signal_create(1, 0, nullptr, &sig);
            if (st != HSA_STATUS_SUCCESS) return hsa_status_to_sf(st);
            void* dst = reinterpret_cast<char*>(segs[i].dst) + off;
            const void* src = reinterpret_cast<const char*>(segs[i].src) + off;
            const uint32_t eng = engines[rr++ % nengines];
            if (eng != 0)
                st = hsa_amd_memory_async_copy_on_engine(dst, cpu, src, gpu, size_t(n), 0, nullptr, sig,
                                                         static_cast<hsa_amd_sdma_engine_id_t>(eng), true);
            else
                st = hsa_amd_memory_async_copy(dst, cpu, src, gpu, size_t(n), 0, nullptr, sig);
            if (st != HSA_STATUS_SUCCESS) {
                hsa_signal_destroy(sig);
                return hsa_status_to_sf(st);
            }
            {
                std::lock_guard<std::mutex> lk(g_dma_mu);
                g_dma.outstanding[sig.handle] = eng;
            }
            signals[(*nsignals)++] = sig.handle;
        }
    }
    return SF_OK;
}

int sf_dma_wait(const uint64_t* signals, int nsignals, uint64_t timeout_ns, uint64_t* start_ns,
                uint64_t* end_ns) {
    if (nsignals < 0 || (nsignals > 0 && signals == nullptr)) return SF_EINVAL;
    // Every copy must be complete before any handle is released, so that a
    // wait that ends at its deadline leaves all of them valid.  Poll with
    // short sleeps: an SDMA completion does not reliably wake a thread
    // blocked in the runtime's interrupt wait (measured: a blocked wait
    // returned 350 ms after the copy had finished).
    // at most ~30 years: the signed duration cannot wrap to a deadline in the past
    const uint64_t capped_ns = timeout_ns < (uint64_t(1) << 60) ? timeout_ns : (uint64_t(1) << 60);
    const auto deadline = std::chrono::steady_clock::now() + std::chrono::nanoseconds(int64_t(capped_ns));
    for (int i = 0; i < nsignals; ++i) {
        if (signals[i] == 0) continue;
        const hsa_signal_t sig{signals[i]};
        while (hsa_signal_load_scacquire(sig) >= 1) {
            if (timeout_ns != 0 && std::chrono::steady_clock::now() >= deadline) return SF_ETIMEDOUT;
            std::this_thread::sleep_for(std::chrono::microseconds(50));
        }
    }
    uint64_t t0 = UINT64_MAX, t1 = 0;
    int rc = SF_OK;
    for (int i = 0; i < nsignals; ++i) {
        if (signals[i] == 0) continue;
        hsa_signal_t sig{signals[i]};
        if (start_ns != nullptr && end_ns != nullptr) {
            hsa_amd_profiling_async_copy_time_t tm;
            if (hsa_amd_profiling_get_async_copy_time(sig, &tm) == HSA_STATUS_SUCCESS && tm.end > 0) {
                if (tm.start < t0) t0 = tm.start;
                if (tm.end > t1) t1 = tm.end;
            }
        }
        {
            // forget the copy before its signal handle can be reused
            std::lock_guard<std::mutex> lk(g_dma_mu);
            g_dma.outstanding.erase(signals[i]);
        }
        hsa_status_t st = hsa_signal_destroy(sig);
        if (st != HSA_STATUS_SUCCESS && rc == SF_OK) rc = hsa_status_to_sf(st);
    }
    if (start_ns != nullptr && end_ns != nullptr) {
        if (t0 == UINT64_MAX || g_dma.ts_freq == 0) {
            *start_ns = *end_ns = 0;
        } else {
            // system timestamp ticks -> ns on the same clock
            const long double scale = 1e9L / (long double)g_dma.ts_freq;
            *start_ns = uint64_t((long double)t0 * scale);
            *end_ns = uint64_t((long double)t1 * scale);
        }
    }
    return rc;
}

int sf_dma_query(const uint64_t* signals, int nsignals, int* done) {
    if (done == nullptr || nsignals < 0 || (nsignals > 0 && signals == nullptr)) return SF_EINVAL;
    *done = 1;
    for (int i = 0; i < nsignals; ++i) {
        if (signals[i] == 0) continue;
        if (hsa_signal_load_scacquire(hsa_signal_t{signals[i]}) >= 1) {
            *done = 0;
            break;
        }
    }
    return SF_OK;
}

int sf_dma_clock_ns(uint64_t* ns) {
    if (ns == nullptr) return SF_EINVAL;
    uint64_t freq = 0;
    {
        std::lock_guard<std::mutex> lk(g_dma_mu);
        if (!g_dma.ok || g_dma.ts_freq == 0) return SF_EINVAL;
        freq = g_dma.ts_freq;
    }
    uint64_t ticks = 0;
    const hsa_status_t st = hsa_system_get_info(HSA_SYSTEM_INFO_TIMESTAMP, &ticks);
    if (st != HSA_STATUS_SUCCESS) return hsa_status_to_sf(st);
    *ns = uint64_t((long double)ticks * (1e9L / (long double)freq));
    return SF_OK;
}

int sf_dma_enable_timing(int on) {
    if (!g_dma.ok) return SF_EINVAL;
    return hsa_status_to_sf(hsa_amd_profiling_async_copy_enable(on != 0));
}

}  // extern "C"
