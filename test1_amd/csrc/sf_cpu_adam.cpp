// Host AdamW for LayerAdam: fp32 params and moments, fp32, bf16 or fp16 grads
// (the row-wise update: fp32 or bf16).
//
// The update is bound by host DRAM bandwidth (26 bytes per element with bf16
// grads: read p, g, m, v and write p, m, v; 28 when it also writes the bf16
// copy of p that bf16 H2D streams), so the kernel is a single streaming pass
// with 512-bit loads/stores over 32K-element chunks that an OpenMP team takes
// dynamically.  Reading bf16 grads directly
// removes the `grad.float()` temporary of the reference
// (optimizer/layer_adam/layer_adam.py:404): bf16 -> fp32 widening is a
// 16-bit left shift and exact, so the update is identical.
//
// Per element, the operation order is that of Adam_Optimizer::Step_AVX,
// optimizer/layer_adam/csrc/cpu_adam.h:170-191 (each step one IEEE
// correctly rounded operation):
//   [L2 mode, wd > 0]  g = fma(p, wd, g)
//   m = m * b1;        m = fma(g, 1 - b1, m)
//   v = v * b2;        g2 = g * g;        v = fma(g2, 1 - b2, v)
//   d = fma(sqrt(v), bc2, eps);           u = m / d
//   [AdamW, wd > 0]    p = fma(p, -lr * wd, p)
//   p = fma(u, step_size, p)              (step_size = -lr / bc1)
// The last (n mod 16) elements of each call are the reference's scalar tail
// (cpu_adam_impl.cpp:39-65), which its compiler contracts differently:
//   m = fma(m, b1, g * (1 - b1)),  v = fma(v, b2, (g * g) * (1 - b2))
// (read from the reference built from source with this toolchain's g++);
// adam_one_tail() reproduces that, so results match it bit for bit for
// equal scalars on every element.

#include <immintrin.h>
#include <omp.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include "../../include/slidefsdp.h"

namespace {

struct Scalars {
    float b1, b2, b1m1, b2m1, eps, bc2, step_size, decay;  // decay: -lr*wd (AdamW) or wd (L2)
    bool use_decay, adamw;
};

Scalars make_scalars(const sf_adam_hparams& h) {
    Scalars c;
    c.b1 = h.beta1;
    c.b2 = h.beta2;
    c.b1m1 = 1.0f - h.beta1;
    c.b2m1 = 1.0f - h.beta2;
    c.eps = h.eps;
    c.bc2 = h.bias_correction2;
    c.step_size = h.step_size;
    c.adamw = h.adamw_mode != 0;
    c.use_decay = h.weight_decay > 0.0f;
    c.decay = c.adamw ? (-1.0f * h.lr * h.weight_decay) : h.weight_decay;
    return c;
}

// fp32 -> bf16, round to nearest even on the bit pattern, NaN -> 0xFFFF: the
// arithmetic of the device staging cast (and of torch's vectorised CPU cast).
inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFu;
    return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

inline float bf16_to_f32(uint16_t b) {
    uint32_t u = uint32_t(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// One element, scalar.  std::fma is correctly rounded whether it becomes an
// instruction or a libm call; no expression here is left for the compiler
// to contract (the file is built with -ffp-contract=off).
inline void adam_one(float& p, float g, float& m, float& v, const Scalars& c) {
    if (c.use_decay && !c.adamw) g = std::fma(p, c.decay, g);
    m = m * c.b1;
    m = std::fma(g, c.b1m1, m);
    v = v * c.b2;
    const float g2 = g * g;
    v = std::fma(g2, c.b2m1, v);
    const float d = std::fma(std::sqrt(v), c.bc2, c.eps);
    const float u = m / d;
    if (c.use_decay && c.adamw) p = std::fma(p, c.decay, p);
    p = std::fma(u, c.step_size, p);
}

// The reference's scalar tail, same steps with the two moment updates fused
// the other way round.
inline void adam_one_tail(float& p, float g, float& m, float& v, const Scalars& c) {
    if (c.use_decay && !c.adamw) g = std::fma(p, c.decay, g);
    m = std::fma(m, c.b1, g * c.b1m1);
    const float g2 = g * g;
    v = std::fma(v, c.b2, g2 * c.b2m1);
    const float d = std::fma(std::sqrt(v), c.bc2, c.eps);
    const float u = m / d;
    if (c.use_decay && c.adamw) p = std::fma(p, c.decay, p);
    p = std::fma(u, c.step_size, p);
}

// fp16 -> fp32, exact (every fp16 value is an fp32 value): the widening of
// `grad.float()` for fp16 units.  A signaling NaN comes back quiet, as the
// hardware conversion gives it.
inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t u;
    if (e == 0x1Fu) {
        u = sign | 0x7F800000u | (m << 13) | (m ? 0x400000u : 0u);
    } else if (e != 0) {
        u = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        u = sign;
    } else {
        // subnormal: m x 2^-24, renormalised
        uint32_t mm = m, ee = 113u;
        while ((mm & 0x400u) == 0) {
            mm <<= 1;
            --ee;
        }
        u = sign | (ee << 23) | ((mm & 0x3FFu) << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

template <int GDT>
inline float load_grad(const void* g, size_t i) {
    if (GDT == SF_DTYPE_BF16) return bf16_to_f32(static_cast<const uint16_t*>(g)[i]);
    if (GDT == SF_DTYPE_F16) return f16_to_f32(static_cast<const uint16_t*>(g)[i]);
    return static_cast<const float*>(g)[i];
}

template <int GDT>
void adam_range_scalar(float* p, const void* g, float* m, float* v, size_t b, size_t e,
                       const Scalars& c, uint16_t* pb) {
    for (size_t i = b; i < e; ++i) {
        adam_one(p[i], load_grad<GDT>(g, i), m[i], v[i], c);
        if (pb) pb[i] = f32_to_bf16_rne(p[i]);
    }
}

template <int GDT>
void adam_range_tail(float* p, const void* g, float* m, float* v, size_t b, size_t e,
                     const Scalars& c, uint16_t* pb) {
    for (size_t i = b; i < e; ++i) {
        adam_one_tail(p[i], load_grad<GDT>(g, i), m[i], v[i], c);
        if (pb) pb[i] = f32_to_bf16_rne(p[i]);
    }
}

// 16 fp32 -> 16 bf16 (RNE, NaN -> 0xFFFF), integer arithmetic in 512-bit lanes.
__attribute__((target("avx512f,avx512bw"))) inline __m256i rne16(__m512 x) {
    const __m512i u = _mm512_castps_si512(x);
    const __m512i lsb = _mm512_and_si512(_mm512_srli_epi32(u, 16), _mm512_set1_epi32(1));
    const __m512i r = _mm512_srli_epi32(_mm512_add_epi32(_mm512_add_epi32(u, _mm512_set1_epi32(0x7FFF)), lsb), 16);
    const __mmask16 nan = _mm512_cmpgt_epu32_mask(_mm512_and_si512(u, _mm512_set1_epi32(0x7FFFFFFF)),
                                                  _mm512_set1_epi32(0x7F800000));
    const __m512i out = _mm512_mask_mov_epi32(r, nan, _mm512_set1_epi32(0xFFFF));
    return _mm512_cvtepi32_epi16(out);
}

template <int GDT>
__attribute__((target("avx512f,avx512bw"))) void adam_range_avx512(float* p, const void* g, float* m,
                                                                    float* v, size_t b, size_t e,
                                                                    const Scalars& c, uint16_t* pb) {
    const __m512 b1 = _mm512_set1_ps(c.b1), b2 = _mm512_set1_ps(c.b2);
    const __m512 b1m1 = _mm512_set1_ps(c.b1m1), b2m1 = _mm512_set1_ps(c.b2m1);
    const __m512 eps = _mm512_set1_ps(c.eps), bc2 = _mm512_set1_ps(c.bc2);
    const __m512 ss = _mm512_set1_ps(c.step_size), dec = _mm512_set1_ps(c.decay);
    const bool l2 = c.use_decay && !c.adamw, dw = c.use_decay && c.adamw;
    // The bf16 copy is only read later by a DMA engine: stream it past the
    // caches (no read-for-ownership) when the 32-byte stores are aligned.
    const bool pb_nt = pb && (reinterpret_cast<uintptr_t>(pb + b) & 31) == 0;
    size_t i = b;
    for (; i + 16 <= e; i += 16) {
        __m512 gv;
        if (GDT == SF_DTYPE_BF16) {
            const __m256i h = _mm256_loadu_si256(
                reinterpret_cast<const __m256i*>(static_cast<const uint16_t*>(g) + i));
            gv = _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(h), 16));
        } else if (GDT == SF_DTYPE_F16) {
            gv = _mm512_cvtph_ps(_mm256_loadu_si256(
                reinterpret_cast<const __m256i*>(static_cast<const uint16_t*>(g) + i)));
        } else {
            gv = _mm512_loadu_ps(static_cast<const float*>(g) + i);
        }
        __m512 mv = _mm512_loadu_ps(m + i);
        __m512 vv = _mm512_loadu_ps(v + i);
        __m512 pv = _mm512_loadu_ps(p + i);
        if (l2) gv = _mm512_fmadd_ps(pv, dec, gv);
        mv = _mm512_mul_ps(mv, b1);
        mv = _mm512_fmadd_ps(gv, b1m1, mv);
        vv = _mm512_mul_ps(vv, b2);
        gv = _mm512_mul_ps(gv, gv);
        vv = _mm512_fmadd_ps(gv, b2m1, vv);
        __m512 d = _mm512_fmadd_ps(_mm512_sqrt_ps(vv), bc2, eps);
        d = _mm512_div_ps(mv, d);
        if (dw) pv = _mm512_fmadd_ps(pv, dec, pv);
        pv = _mm512_fmadd_ps(d, ss, pv);
        _mm512_storeu_ps(p + i, pv);
        _mm512_storeu_ps(m + i, mv);
        _mm512_storeu_ps(v + i, vv);
        if (pb_nt) _mm256_stream_si256(reinterpret_cast<__m256i*>(pb + i), rne16(pv));
        else if (pb) _mm256_storeu_si256(reinterpret_cast<__m256i*>(pb + i), rne16(pv));
    }
    if (pb_nt) _mm_sfence();
    adam_range_scalar<GDT>(p, g, m, v, i, e, c, pb);
}

bool host_has_avx512() {
    static const bool has = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw");
    return has;
}

int g_threads = 0;  // <= 0: OpenMP default

__attribute__((target("avx512f,avx512bw"))) void cast_range_avx512(const float* src, uint16_t* dst,
                                                                    size_t b, size_t e) {
    size_t i = b;
    for (; i + 16 <= e; i += 16) _mm256_storeu_si256(reinterpret_cast<__m256i*>(dst + i), rne16(_mm512_loadu_ps(src + i)));
    for (; i < e; ++i) dst[i] = f32_to_bf16_rne(src[i]);
}

template <int GDT>
void adam_parallel(float* p, const void* g, float* m, float* v, size_t n, const Scalars& c,
                   uint16_t* pb) {
    const bool avx = host_has_avx512();
    const size_t n_main = n & ~size_t(15);  // elements before the reference's scalar tail
    int nt = g_threads > 0 ? g_threads : omp_get_max_threads();
    // Small updates do not pay for a team: ~1 MiB of traffic per thread minimum.
    const size_t min_per_thread = size_t(1) << 16;
    if (size_t(nt) * min_per_thread > n) nt = int(n / min_per_thread) > 0 ? int(n / min_per_thread) : 1;
    // Chunks of 32K elements (~0.9 MB of traffic) handed out dynamically: a
    // thread that the OS preempts (the host also feeds the GPU) takes fewer
    // chunks instead of stalling the whole update.  Each element's result
    // depends only on its position, so the partition does not change bits.
    const size_t chunk = size_t(1) << 15;
    const long nchunks = long((n + chunk - 1) / chunk);
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
    for (long k = 0; k < nchunks; ++k) {
        const size_t b = size_t(k) * chunk;
        const size_t e = std::min(n, b + chunk);
        const size_t em = std::min(e, n_main);
        if (b < em) {
            if (avx) adam_range_avx512<GDT>(p, g, m, v, b, em, c, pb);
            else adam_range_scalar<GDT>(p, g, m, v, b, em, c, pb);
        }
        if (std::max(b, n_main) < e) adam_range_tail<GDT>(p, g, m, v, std::max(b, n_main), e, c, pb);
    }
}

// Per-optimizer running state of beta1^t / beta2^t and the bias
// corrections, as Adam_Optimizer keeps it (cpu_adam.h:57-89): the powers
// advance by one float multiply when calls arrive with consecutive step
// numbers and are recomputed with pow() otherwise, and a change of betas
// resets them.
struct AdamState {
    float alpha, beta1, beta2, eps, weight_decay;
    float beta1_t = 1.0f, beta2_t = 1.0f;
    size_t step = 0;
    bool adamw;
    std::mutex mu;

    void increment_step(size_t t, float b1, float b2) {
        if (b1 != beta1 || b2 != beta2) {
            step = t;
            beta1 = b1;
            beta2 = b2;
            beta1_t = float(std::pow(double(beta1), double(t)));
            beta2_t = float(std::pow(double(beta2), double(t)));
        } else {
            ++step;
            if (step != t) {
                beta1_t = float(std::pow(double(beta1), double(t)));
                beta2_t = float(std::pow(double(beta2), double(t)));
                step = t;
            } else {
                beta1_t *= beta1;
                beta2_t *= beta2;
            }
        }
    }
};

std::mutex g_registry_mu;
std::unordered_map<int, std::shared_ptr<AdamState>> g_registry;

std::shared_ptr<AdamState> find_state(int id) {
    std::lock_guard<std::mutex> lk(g_registry_mu);
    auto it = g_registry.find(id);
    return it == g_registry.end() ? nullptr : it->second;
}

}  // namespace

extern "C" {

const char* sf_error_string(int status) {
    switch (status) {
        case SF_OK: return "success";
        case SF_EINVAL: return "sf: invalid argument (null pointer, bad size or enum)";
        case SF_EDTYPE: return "sf: dtype combination not supported";
        case SF_ENOOPT: return "sf: unknown optimizer id";
        case SF_ENOREQ: return "sf: unknown or already released I/O ticket";
        case SF_EALIGN: return "sf: O_DIRECT transfer: buffer, size and offset must be multiples of SF_IO_ALIGN";
        default: break;
    }
    if (status > SF_EIO_BASE && status < SF_EIO_BASE + 4096) {
        // strerror_r (GNU) may return a static string or fill the buffer.
        static thread_local char buf[160];
        char msg[128];
        const char* e = strerror_r(status - SF_EIO_BASE, msg, sizeof msg);
        snprintf(buf, sizeof buf, "sf: file I/O failed: %s", e);
        return buf;
    }
    return "sf: unknown status";
}

int sf_abi_version(void) { return SF_ABI_VERSION; }

int sf_cpu_set_threads(int nthreads) {
    g_threads = nthreads;
    return SF_OK;
}

int sf_cpu_has_avx512(void) { return host_has_avx512() ? 1 : 0; }

int sf_cpu_adam_step_cast(float* params, const void* grads, int g_dtype, float* exp_avg,
                          float* exp_avg_sq, uint16_t* params_bf16, size_t n, const sf_adam_hparams* hp) {
    if (n == 0) return SF_OK;
    if (!params || !grads || !exp_avg || !exp_avg_sq || !hp) return SF_EINVAL;
    const Scalars c = make_scalars(*hp);
    switch (g_dtype) {
        case SF_DTYPE_F32: adam_parallel<SF_DTYPE_F32>(params, grads, exp_avg, exp_avg_sq, n, c, params_bf16); break;
        case SF_DTYPE_BF16: adam_parallel<SF_DTYPE_BF16>(params, grads, exp_avg, exp_avg_sq, n, c, params_bf16); break;
        case SF_DTYPE_F16: adam_parallel<SF_DTYPE_F16>(params, grads, exp_avg, exp_avg_sq, n, c, params_bf16); break;
        default: return SF_EDTYPE;
    }
    return SF_OK;
}

int sf_cpu_adam_step(float* params, const void* grads, int g_dtype, float* exp_avg,
                     float* exp_avg_sq, size_t n, const sf_adam_hparams* hp) {
    return sf_cpu_adam_step_cast(params, grads, g_dtype, exp_avg, exp_avg_sq, nullptr, n, hp);
}

int sf_cpu_cast_f32_bf16(const float* src, uint16_t* dst, size_t n) {
    if (n == 0) return SF_OK;
    if (!src || !dst) return SF_EINVAL;
    const bool avx = host_has_avx512();
    int nt = g_threads > 0 ? g_threads : omp_get_max_threads();
    const size_t min_per_thread = size_t(1) << 18;
    if (size_t(nt) * min_per_thread > n) nt = int(n / min_per_thread) > 0 ? int(n / min_per_thread) : 1;
#pragma omp parallel num_threads(nt)
    {
        const int t = omp_get_thread_num(), T = omp_get_num_threads();
        const size_t blocks = (n + 127) / 128;
        const size_t b = std::min(n, (blocks * size_t(t) / size_t(T)) * 128);
        const size_t e = std::min(n, (blocks * size_t(t + 1) / size_t(T)) * 128);
        if (avx) cast_range_avx512(src, dst, b, e);
        else for (size_t i = b; i < e; ++i) dst[i] = f32_to_bf16_rne(src[i]);
    }
    return SF_OK;
}

int sf_adam_create(int optimizer_id, float alpha, float beta1, float beta2, float eps,
                   float weight_decay, int adamw_mode, int should_log) {
    auto st = std::make_shared<AdamState>();
    st->alpha = alpha;
    st->beta1 = beta1;
    st->beta2 = beta2;
    st->eps = eps;
    st->weight_decay = weight_decay;
    st->adamw = adamw_mode != 0;
    {
        std::lock_guard<std::mutex> lk(g_registry_mu);
        g_registry[optimizer_id] = st;
    }
    if (should_log) {
        std::printf("Adam Optimizer #%d is created with %s arithmetic capability.\n", optimizer_id,
                    host_has_avx512() ? "AVX512" : "scalar");
        std::printf("Config: alpha=%f, betas=(%f, %f), weight_decay=%f, adam_w=%d\n", alpha, beta1,
                    beta2, weight_decay, adamw_mode != 0 ? 1 : 0);
        std::fflush(stdout);
    }
    return SF_OK;
}

int sf_adam_update_cast(int optimizer_id, size_t step, float lr, float beta1, float beta2, float eps,
                        float weight_decay, int bias_correction, float* params, const void* grads,
                        int g_dtype, float* exp_avg, float* exp_avg_sq, uint16_t* params_bf16, size_t n);

int sf_adam_update(int optimizer_id, size_t step, float lr, float beta1, float beta2, float eps,
                   float weight_decay, int bias_correction, float* params, const void* grads,
                   int g_dtype, float* exp_avg, float* exp_avg_sq, size_t n) {
    return sf_adam_update_cast(optimizer_id, step, lr, beta1, beta2, eps, weight_decay, bias_correction,
                               params, grads, g_dtype, exp_avg, exp_avg_sq, nullptr, n);
}

}  // extern "C"

namespace {

// The scalars of one stateful update (cpu_adam.h:57-89, 108-141): advance the
// optimizer's beta powers for ``step`` and derive the bias corrections.
void stateful_hparams(AdamState& stt, size_t step, float lr, float beta1, float beta2, float eps,
                      float weight_decay, int bias_correction, sf_adam_hparams& hp) {
    AdamState* st = &stt;
    {
        std::lock_guard<std::mutex> lk(st->mu);
        st->increment_step(step, beta1, beta2);
        st->alpha = lr;
        st->eps = eps;
        st->weight_decay = weight_decay;
        float bc1 = 1.0f, bc2 = 1.0f;
        if (bias_correction) {
            // All in float, as cpu_adam.h:86-87 compiles (sqrt of a float
            // resolves to the float overload there; pinned against the
            // compiled reference).
            bc1 = 1.0f - st->beta1_t;
            bc2 = 1.0f / std::sqrt(1.0f - st->beta2_t);
        }
        hp.beta1 = st->beta1;
        hp.beta2 = st->beta2;
        hp.eps = eps;
        hp.weight_decay = weight_decay;
        hp.lr = lr;
        hp.step_size = -1.0f * lr / bc1;
        hp.bias_correction2 = bc2;
        hp.adamw_mode = st->adamw ? 1 : 0;
    }
}

// Scalars of one update as the reference's call sequence yields them when
// every unit is stepped once per step, last unit first, each with at least
// two calls in all per step (Adam_Optimizer::IncrementStep, cpu_adam.h:57-76,
// then cpu_adam.h:77-89): the first call of step t multiplies the beta^(t-1)
// that the previous step's calls left (float(pow) after its second call, 1
// before the first step) by beta; every later call of the step recomputes
// beta^t with pow.  The caller says which call is the first.
void hparams_in_reference_order(size_t step, float lr, float beta1, float beta2, float eps, float weight_decay,
                                int bias_correction, int adamw_mode, int first_of_step, sf_adam_hparams& hp) {
    float b1t, b2t;
    if (first_of_step) {
        const float p1 = step > 1 ? float(std::pow(double(beta1), double(step - 1))) : 1.0f;
        const float p2 = step > 1 ? float(std::pow(double(beta2), double(step - 1))) : 1.0f;
        b1t = p1 * beta1;
        b2t = p2 * beta2;
    } else {
        b1t = float(std::pow(double(beta1), double(step)));
        b2t = float(std::pow(double(beta2), double(step)));
    }
    float bc1 = 1.0f, bc2 = 1.0f;
    if (bias_correction) {
        bc1 = 1.0f - b1t;
        bc2 = 1.0f / std::sqrt(1.0f - b2t);
    }
    hp.beta1 = beta1;
    hp.beta2 = beta2;
    hp.eps = eps;
    hp.weight_decay = weight_decay;
    hp.lr = lr;
    hp.step_size = -1.0f * lr / bc1;
    hp.bias_correction2 = bc2;
    hp.adamw_mode = adamw_mode ? 1 : 0;
}

// Rows of a [n_rows, row_len] tensor; row r takes its gradient from
// grads[row_slot[r]] or, for row_slot[r] < 0, zeros.  row_len is a multiple
// of 16, so every row starts a 16-element group and no element falls in the
// reference's scalar tail: each element gets exactly the dense update.
template <int GDT>
void adam_rows(float* p, float* m, float* v, uint16_t* pb, size_t n_rows, size_t row_len,
               const int64_t* row_slot, const void* grads, const Scalars& c) {
    using G = typename std::conditional<GDT == SF_DTYPE_BF16, uint16_t, float>::type;
    const G* g = static_cast<const G*>(grads);
    std::vector<G> zeros(row_len, G(0));
    const bool avx = host_has_avx512();
    int nt = g_threads > 0 ? g_threads : omp_get_max_threads();
    const long rows_per_chunk = long(std::max<size_t>(1, (size_t(1) << 15) / row_len));
    const long nchunks = long((n_rows + rows_per_chunk - 1) / rows_per_chunk);
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
    for (long k = 0; k < nchunks; ++k) {
        const size_t r0 = size_t(k) * rows_per_chunk, r1 = std::min(n_rows, r0 + size_t(rows_per_chunk));
        for (size_t r = r0; r < r1; ++r) {
            if (row_slot[r] == SF_ROW_SKIP) continue;
            const size_t o = r * row_len;
            const G* gr = row_slot[r] >= 0 ? g + size_t(row_slot[r]) * row_len : zeros.data();
            uint16_t* pbr = pb ? pb + o : nullptr;
            if (avx) adam_range_avx512<GDT>(p + o, gr, m + o, v + o, 0, row_len, c, pbr);
            else adam_range_scalar<GDT>(p + o, gr, m + o, v + o, 0, row_len, c, pbr);
        }
    }
}

}  // namespace

extern "C" {

int sf_adam_update_cast(int optimizer_id, size_t step, float lr, float beta1, float beta2, float eps,
                        float weight_decay, int bias_correction, float* params, const void* grads,
                        int g_dtype, float* exp_avg, float* exp_avg_sq, uint16_t* params_bf16, size_t n) {
    std::shared_ptr<AdamState> st = find_state(optimizer_id);
    if (!st) return SF_ENOOPT;
    if (g_dtype != SF_DTYPE_F32 && g_dtype != SF_DTYPE_BF16 && g_dtype != SF_DTYPE_F16) return SF_EDTYPE;
    if (n > 0 && (!params || !grads || !exp_avg || !exp_avg_sq)) return SF_EINVAL;
    sf_adam_hparams hp;
    stateful_hparams(*st, step, lr, beta1, beta2, eps, weight_decay, bias_correction, hp);
    return sf_cpu_adam_step_cast(params, grads, g_dtype, exp_avg, exp_avg_sq, params_bf16, n, &hp);
}

int sf_adam_update_rows(int optimizer_id, size_t step, float lr, float beta1, float beta2, float eps,
                        float weight_decay, int bias_correction, float* params, float* exp_avg,
                        float* exp_avg_sq, uint16_t* params_bf16, size_t n_rows, size_t row_len,
                        const int64_t* row_slot, const void* grads, size_t n_grad_rows, int g_dtype) {
    std::shared_ptr<AdamState> st = find_state(optimizer_id);
    if (!st) return SF_ENOOPT;
    if (g_dtype != SF_DTYPE_F32 && g_dtype != SF_DTYPE_BF16) return SF_EDTYPE;
    if (n_rows == 0 || row_len == 0) return SF_OK;
    if (row_len % 16 != 0) return SF_EINVAL;
    if (!params || !exp_avg || !exp_avg_sq || !row_slot || (n_grad_rows > 0 && !grads)) return SF_EINVAL;
    for (size_t r = 0; r < n_rows; ++r) {
        if (row_slot[r] < SF_ROW_SKIP || (row_slot[r] >= 0 && size_t(row_slot[r]) >= n_grad_rows)) return SF_EINVAL;
    }
    sf_adam_hparams hp;
    stateful_hparams(*st, step, lr, beta1, beta2, eps, weight_decay, bias_correction, hp);
    const Scalars c = make_scalars(hp);
    if (g_dtype == SF_DTYPE_BF16) adam_rows<SF_DTYPE_BF16>(params, exp_avg, exp_avg_sq, params_bf16, n_rows, row_len, row_slot, grads, c);
    else adam_rows<SF_DTYPE_F32>(params, exp_avg, exp_avg_sq, params_bf16, n_rows, row_len, row_slot, grads, c);
    return SF_OK;
}

int sf_adam_hparams_in_order(size_t step, float lr, float beta1, float beta2, float eps, float weight_decay,
                             int bias_correction, int adamw_mode, int first_of_step, sf_adam_hparams* hp) {
    if (!hp || step == 0) return SF_EINVAL;
    hparams_in_reference_order(step, lr, beta1, beta2, eps, weight_decay, bias_correction, adamw_mode,
                               first_of_step, *hp);
    return SF_OK;
}

int sf_cpu_adam_step_rows(float* params, float* exp_avg, float* exp_avg_sq, uint16_t* params_bf16,
                          size_t n_rows, size_t row_len, const int64_t* row_slot, const void* grads,
                          size_t n_grad_rows, int g_dtype, const sf_adam_hparams* hp) {
    if (g_dtype != SF_DTYPE_F32 && g_dtype != SF_DTYPE_BF16) return SF_EDTYPE;
    if (n_rows == 0 || row_len == 0) return SF_OK;
    if (row_len % 16 != 0) return SF_EINVAL;
    if (!hp || !params || !exp_avg || !exp_avg_sq || !row_slot || (n_grad_rows > 0 && !grads)) return SF_EINVAL;
    for (size_t r = 0; r < n_rows; ++r) {
        if (row_slot[r] < SF_ROW_SKIP || (row_slot[r] >= 0 && size_t(row_slot[r]) >= n_grad_rows)) return SF_EINVAL;
    }
    const Scalars c = make_scalars(*hp);
    if (g_dtype == SF_DTYPE_BF16) adam_rows<SF_DTYPE_BF16>(params, exp_avg, exp_avg_sq, params_bf16, n_rows, row_len, row_slot, grads, c);
    else adam_rows<SF_DTYPE_F32>(params, exp_avg, exp_avg_sq, params_bf16, n_rows, row_len, row_slot, grads, c);
    return SF_OK;
}

int sf_adam_destroy(int optimizer_id) {
    std::lock_guard<std::mutex> lk(g_registry_mu);
    g_registry.erase(optimizer_id);
    return SF_OK;
}

}  // extern "C"
