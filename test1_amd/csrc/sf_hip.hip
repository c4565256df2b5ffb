// Device side of the layer-streaming path for MI355X (gfx950).
//
// Every kernel here is a streaming kernel: each byte is read once and
// written once, so the bound is HBM bandwidth (or the host link, for the
// copies), never the matrix cores.  The kernels therefore use
//   - 128-bit global loads and stores, 8 elements per lane per group,
//   - several independent groups per lane to keep enough bytes in flight,
//   - 256-lane workgroups (4 wave64s) and an exact grid of many thousands
//     of workgroups so all 256 CUs over the 8 XCDs stay busy,
//   - no LDS and no MFMA.
//
// The C ABI is declared in include/slidefsdp.h.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/slidefsdp.h"

namespace {

constexpr int kThreads = 256;  // lanes per workgroup (4 wave64s)
constexpr int kUnroll = 4;     // 8-element groups per lane per workgroup tile
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

// ---------------------------------------------------------------------
// Flat cast: n8 groups of 8 elements, both pointers 16-byte aligned.
// Workgroup b owns groups [b*kThreads*kUnroll, (b+1)*kThreads*kUnroll);
// within it, unroll step k covers one contiguous run of kThreads groups,
// so every load/store instruction of a wave touches one contiguous
// 1 KiB (fp32 half-group) or 1 KiB (bf16 group) span.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void cast_flat_kernel(
    const float* __restrict__ src, uint16_t* __restrict__ dst, uint64_t n8) {
    const uint64_t tile0 = uint64_t(blockIdx.x) * (kThreads * kUnroll);
    if (tile0 + kThreads * kUnroll <= n8) {
        // Full tile (every workgroup but possibly the last): all 2*kUnroll
        // loads are issued before the first conversion, with no per-lane
        // predicate between them, so each lane has 128 bytes in flight.
        f32x4 a[kUnroll], b[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) {
            const f32x4* p = reinterpret_cast<const f32x4*>(src + (tile0 + k * kThreads + threadIdx.x) * kGroup);
            a[k] = __builtin_nontemporal_load(p);
            b[k] = __builtin_nontemporal_load(p + 1);
        }
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) {
            __builtin_nontemporal_store(cast8(a[k], b[k]),
                reinterpret_cast<u32x4*>(dst + (tile0 + k * kThreads + threadIdx.x) * kGroup));
        }
    } else {
        for (int k = 0; k < kUnroll; ++k) {
            const uint64_t g = tile0 + k * kThreads + threadIdx.x;
            if (g < n8) {
                const f32x4* p = reinterpret_cast<const f32x4*>(src + g * kGroup);
                __builtin_nontemporal_store(cast8(p[0], p[1]), reinterpret_cast<u32x4*>(dst + g * kGroup));
            }
        }
    }
}

// Scalar cast for tails and for pointers that are not 16-byte aligned.
__global__ __launch_bounds__(kThreads) void cast_scalar_kernel(
    const float* __restrict__ src, uint16_t* __restrict__ dst, uint64_t n) {
    const uint64_t stride = uint64_t(gridDim.x) * kThreads;
    for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
        dst[i] = uint16_t(rne_bf16(__float_as_uint(src[i])));
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

extern "C" {

const char* sf_error_string(int status) {
    switch (status) {
        case SF_OK: return "success";
        case SF_EINVAL: return "sf: invalid argument (null pointer, bad size or enum)";
        case SF_ETOOMANY: return "sf: too many segments for one call";
        case SF_EDTYPE: return "sf: dtype combination not supported";
        case SF_ENOOPT: return "sf: unknown optimizer id";
        case SF_EOVERLAP: return "sf: source and destination overlap";
        default: return hipGetErrorString(hipError_t(status));
    }
}

int sf_abi_version(void) { return 1; }

int sf_cast_f32_bf16(const float* src, uint16_t* dst, size_t n, sf_stream_t stream) {
    if (n == 0) return SF_OK;
    if (src == nullptr || dst == nullptr) return SF_EINVAL;
    const uintptr_t s = reinterpret_cast<uintptr_t>(src), d = reinterpret_cast<uintptr_t>(dst);
    // fp32 source [s, s+4n) and bf16 destination [d, d+2n) must not overlap:
    // workgroups run in no particular order.
    if (s < d + 2 * n && d < s + 4 * n) return SF_EOVERLAP;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const uint64_t n8 = ((s | d) & 15) == 0 ? n / kGroup : 0;
    if (n8 > 0) {
        const uint64_t blocks = ceil_div(n8, uint64_t(kThreads) * kUnroll);
        if (blocks > kMaxBlocks) return SF_EINVAL;
        hipLaunchKernelGGL(cast_flat_kernel, dim3(uint32_t(blocks)), dim3(kThreads), 0, st, src, dst, n8);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return int(e);
    }
    const uint64_t done = n8 * kGroup;
    if (done < n) {
        const uint64_t rest = n - done;
        uint64_t blocks = ceil_div(rest, kThreads);
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(cast_scalar_kernel, dim3(uint32_t(blocks)), dim3(kThreads), 0, st,
                           src + done, dst + done, rest);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return int(e);
    }
    return SF_OK;
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
    return int(hipMemcpyAsync(dst, src, bytes, k, reinterpret_cast<hipStream_t>(stream)));
}

int sf_host_alloc(void** out, size_t bytes) {
    if (out == nullptr) return SF_EINVAL;
    *out = nullptr;
    if (bytes == 0) return SF_OK;
    return int(hipHostMalloc(out, bytes, hipHostMallocDefault));
}

int sf_host_free(void* ptr) {
    if (ptr == nullptr) return SF_OK;
    return int(hipHostFree(ptr));
}

int sf_host_device_pointer(void* host_ptr, void** device_ptr) {
    if (host_ptr == nullptr || device_ptr == nullptr) return SF_EINVAL;
    *device_ptr = nullptr;
    return int(hipHostGetDevicePointer(device_ptr, host_ptr, 0));
}

}  // extern "C"
