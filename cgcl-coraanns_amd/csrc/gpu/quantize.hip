// RaBitQ quantisation of index rows on the GPU (index build), bit-identical to the host
// builder (csrc/host/index.cpp, which restates rabitq_impl.hpp:76-137 one_bit_code_with_factor,
// 276-333 best_rescale_factor, 336-360 quantize_ex and 405-500 ex_bits_code_with_factor).
//
// One wave per row. Every double-precision sum the host builder forms sequentially in
// index order (the dot products, the initial numerator of the rescale search, ipnorm) is
// formed by lane 0 in the same order, so its roundings are the same; float expressions are
// evaluated term by term as written there (contraction off), and t * |o| + 1e-5 is one
// fused multiply-add, as the host compiler emits it (and std::fma makes explicit).
//
// best_rescale_factor sweeps t upward through the points where some coordinate's code
// increments, in (t, coordinate) order, keeping the t that maximises
// <code + 1/2, |o|> / ||code + 1/2||. Here the sweep runs over windows of t: for each window
// the lanes enumerate their coordinates' increments inside it (integer ranges found with the
// same double divisions that define each t), the window's events (at most kQzWin) are sorted
// by (t, coordinate) in LDS, and lane 0 applies them in order with the host's updates. A
// window holding too many events is halved; one holding a single value of t has at most one
// event per coordinate (P <= 1024). Events at or above t_end (first increments of tiny
// coordinates) come last, in a window of their own.
#include <float.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <string>

#include "../../../include/cora_gpu.h"
#include "engine_internal.h"

#pragma clang fp contract(off)

namespace cora {
namespace {

constexpr int kQzMaxP = 1024;
constexpr int kQzWin = 1024;          // events per sorted window
constexpr int kQzTarget = 768;        // events per window aimed at
constexpr int kQzCap = 127;           // 2^7 - 1 (7 ex-bits)
constexpr int kQzNEnum = 10;
constexpr double kQzTight = 0.81;     // kTightStart[7] (rabitq_impl.hpp:263-273)
constexpr double kQzEps = 1e-5;
constexpr float kQzConstEpsilon = 1.9f;  // rabitq_impl.hpp:18

struct QzArgs {
    const float *x;        // [rows][P] rotated rows
    const float *cent;     // [nlist][P] rotated centroids
    const uint32_t *assign;  // [rows]
    uint32_t rows, P;
    int metric;
    uint8_t *bits;         // [rows][P/8] sign bits, dimension 8b + j at bit 7 - j of byte b
    float *f1;             // [rows][3] f_add, f_rescale, f_error
    uint8_t *code;         // [rows][P] ex-code values (complemented for negative residuals)
    float *f2;             // [rows][2] f_add_ex, f_rescale_ex
};

__device__ __forceinline__ void qz_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// t of the increment to code value u of a coordinate with |o| = a (the host's
// static_cast<double>(u) / oi)
__device__ __forceinline__ double inc_t(int u, double a) { return (double)u / a; }

// smallest u >= 1 with u / a >= ta (a > 0)
__device__ int u_ceil(double ta, double a) {
    double g = ceil(ta * a);
    int u = g < 1.0 ? 1 : (g > 1e9 ? 1000000000 : (int)g);
    while (u > 1 && inc_t(u - 1, a) >= ta)
        --u;
    while (inc_t(u, a) < ta)
        ++u;
    return u;
}

// largest u >= 0 with u / a < tb (a > 0); 0 when none
__device__ int u_floor(double tb, double a) {
    double g = floor(tb * a);
    int u = g < 0.0 ? 0 : (g > 1e9 ? 1000000000 : (int)g);
    while (u > 0 && !(inc_t(u, a) < tb))
        --u;
    while (inc_t(u + 1, a) < tb)
        ++u;
    return u;
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ uint32_t wave_excl_scan(uint32_t v, uint32_t lane) {
    uint32_t incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o, 64);
        if (lane >= (uint32_t)o)
            incl += y;
    }
    return incl - v;
}

// (t, e) pairs in LDS sorted ascending by t, then by coordinate (e >> 8), bitonic over the
// next power of two (padding +inf), one wave.
__device__ void sort_events(double *s_t, uint32_t *s_e, uint32_t n, uint32_t lane) {
    uint32_t np2 = 1;
    while (np2 < n)
        np2 <<= 1;
    for (uint32_t i = n + lane; i < np2; i += 64) {
        s_t[i] = __longlong_as_double(0x7FF0000000000000ll);
        s_e[i] = 0xFFFFFFFFu;
    }
    qz_sync();
    for (uint32_t size = 2; size <= np2; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = lane; i < np2; i += 64) {
                const uint32_t j = i ^ stride;
                if (j > i) {
                    const bool asc = (i & size) == 0;
                    const double ti = s_t[i], tj = s_t[j];
                    const uint32_t ei = s_e[i], ej = s_e[j];
                    const bool gt = ti > tj || (ti == tj && (ei >> 8) > (ej >> 8));
                    if (gt == asc) {
                        s_t[i] = tj;
                        s_t[j] = ti;
                        s_e[i] = ej;
                        s_e[j] = ei;
                    }
                }
            }
            qz_sync();
        }
    }
}

__global__ __launch_bounds__(64) void quantize_kernel(const QzArgs a) {
    __shared__ float s_o[kQzMaxP], s_c[kQzMaxP], s_abs[kQzMaxP];
    __shared__ uint8_t s_code[kQzMaxP];
    __shared__ double s_t[kQzWin];
    __shared__ uint32_t s_e[kQzWin];
    __shared__ double s_best[2];
    const uint32_t lane = threadIdx.x, P = a.P;
    for (uint32_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
        const float *x = a.x + (size_t)row * P;
        const float *cg = a.cent + (size_t)a.assign[row] * P;
        for (uint32_t i = lane; i < P; i += 64) {
            const float c = cg[i];
            s_c[i] = c;
            s_o[i] = x[i] - c;
        }
        qz_sync();
        // ---- one-bit code and factors (quantize_one_bit) ----
        for (uint32_t b = lane; b < P / 8; b += 64) {
            uint32_t byte = 0;
            for (uint32_t j = 0; j < 8; ++j)
                byte |= (s_o[8 * b + j] > 0.0f ? 1u : 0u) << (7 - j);
            a.bits[(size_t)row * (P / 8) + b] = (uint8_t)byte;
        }
        double oo = 0.0, oc = 0.0;  // dot(o, o), dot(o, c): shared with the ex-code factors
        if (lane == 0) {
            double oxu = 0.0, cxu = 0.0;
            for (uint32_t i = 0; i < P; ++i) {
                const float o = s_o[i], c = s_c[i];
                const float xu = (o > 0.0f ? 1.0f : 0.0f) - 0.5f;
                oo += (double)o * o;
                oxu += (double)o * xu;
                cxu += (double)c * xu;
                oc += (double)o * c;
            }
            const float l2_sqr = (float)oo;
            const float l2 = sqrtf(l2_sqr);
            float ip_resi = (float)oxu;
            const float ip_cent = (float)cxu;
            if (ip_resi == 0.0f)
                ip_resi = INFINITY;
            const float xu_sqr = (float)((double)P * 0.25);
            const float err = l2 * kQzConstEpsilon *
                              sqrtf((((l2_sqr * xu_sqr) / (ip_resi * ip_resi)) - 1.0f) / (float)(P - 1));
            float *f = a.f1 + (size_t)row * 3;
            if (a.metric == 0) {
                f[0] = l2_sqr + (2.0f * l2_sqr * ip_cent / ip_resi);
                f[1] = -2.0f * l2_sqr / ip_resi;
                f[2] = 2.0f * err;
            } else {
                f[0] = 1.0f - (float)oc + (l2_sqr * ip_cent / ip_resi);
                f[1] = -l2_sqr / ip_resi;
                f[2] = err;
            }
        }
        // ---- ex-code (quantize_ex_bits, best_rescale_factor) ----
        const float norm = sqrtf((float)__shfl(oo, 0, 64));
        float mx = 0.0f;
        for (uint32_t i = lane; i < P; i += 64) {
            const float v = fabsf(s_o[i] / norm);
            s_abs[i] = v;
            mx = fmaxf(mx, v);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        qz_sync();
        const double max_o = (double)mx;
        const double t_end = (double)(kQzCap + kQzNEnum) / max_o;
        const double t_start = t_end * kQzTight;
        // per coordinate: initial code c and the last main increment U (main increments are
        // the code values c+1 .. U, all with t < t_end; U = c when the first is not)
        uint32_t nmain = 0;
        double lo = t_end;
        for (uint32_t i = lane; i < P; i += 64) {
            const double ai = (double)s_abs[i];
            const int c = (int)fma(t_start, ai, kQzEps);
            const double t1 = inc_t(c + 1, ai);
            int U = c;
            if (t1 < t_end) {
                U = c + 1;
                if (c + 2 <= kQzCap && inc_t(c + 2, ai) < t_end)
                    U = min(kQzCap, u_floor(t_end, ai));
                lo = fmin(lo, t1);
            }
            nmain += (uint32_t)(U - c);
        }
        nmain = wave_sum_u32(nmain);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            lo = fmin(lo, __shfl_xor(lo, o, 64));
        // lane 0: the initial numerator and denominator, in coordinate order
        double num = 0.0, den = (double)P * 0.25, best_ip = 0.0, best_t = 0.0;
        if (lane == 0) {
            for (uint32_t i = 0; i < P; ++i) {
                const double ai = (double)s_abs[i];
                const int c = (int)fma(t_start, ai, kQzEps);
                den += (double)(c * c + c);
                num += (c + 0.5) * ai;
            }
        }
        // the sweep over one window [ta, tb) of main increments (tb <= t_end), or over the
        // increments at or above t_end (overflow); returns false when it holds more than
        // kQzWin events
        auto window = [&](double ta, double tb, bool overflow) -> bool {
            uint32_t cnt = 0;
            for (uint32_t i = lane; i < P; i += 64) {
                const double ai = (double)s_abs[i];
                const int c = (int)fma(t_start, ai, kQzEps);
                const double t1 = inc_t(c + 1, ai);
                if (overflow) {
                    cnt += t1 >= t_end ? 1u : 0u;
                } else if (t1 < t_end) {
                    const int U = c + 2 <= kQzCap && inc_t(c + 2, ai) < t_end ? min(kQzCap, u_floor(t_end, ai)) : c + 1;
                    const int u0 = max(c + 1, u_ceil(ta, ai)), u1 = min(U, u_floor(tb, ai));
                    cnt += u1 >= u0 ? (uint32_t)(u1 - u0 + 1) : 0u;
                }
            }
            const uint32_t total = wave_sum_u32(cnt);
            if (total > (uint32_t)kQzWin)
                return false;
            if (total == 0)
                return true;
            uint32_t pos = wave_excl_scan(cnt, lane);
            for (uint32_t i = lane; i < P; i += 64) {
                const double ai = (double)s_abs[i];
                const int c = (int)fma(t_start, ai, kQzEps);
                const double t1 = inc_t(c + 1, ai);
                if (overflow) {
                    if (t1 >= t_end) {
                        s_t[pos] = t1;
                        s_e[pos] = (i << 8) | (uint32_t)(c + 1);
                        ++pos;
                    }
                } else if (t1 < t_end) {
                    const int U = c + 2 <= kQzCap && inc_t(c + 2, ai) < t_end ? min(kQzCap, u_floor(t_end, ai)) : c + 1;
                    const int u0 = max(c + 1, u_ceil(ta, ai)), u1 = min(U, u_floor(tb, ai));
                    for (int u = u0; u <= u1; ++u) {
                        s_t[pos] = inc_t(u, ai);
                        s_e[pos] = (i << 8) | (uint32_t)u;
                        ++pos;
                    }
                }
            }
            qz_sync();
            sort_events(s_t, s_e, total, lane);
            if (lane == 0) {
                for (uint32_t k = 0; k < total; ++k) {
                    const uint32_t e = s_e[k];
                    den += (double)(2 * (int)(e & 255u));
                    num += (double)s_abs[e >> 8];
                    const double ip = num / sqrt(den);
                    if (ip > best_ip) {
                        best_ip = ip;
                        best_t = s_t[k];
                    }
                }
            }
            qz_sync();
            return true;
        };
        if (nmain > 0) {
            const uint32_t nwin = (nmain + kQzTarget - 1) / kQzTarget;
            const double width = (t_end - lo) / (double)nwin;
            double ta = lo;
            uint32_t w = 1;
            while (ta < t_end) {
                double tb = w >= nwin ? t_end : fmin(t_end, lo + width * (double)w);
                if (!(tb > ta))
                    tb = t_end;
                while (!window(ta, tb, false)) {
                    double mid = ta + (tb - ta) * 0.5;
                    if (!(mid > ta))
                        mid = nextafter(ta, t_end);  // a single value of t: at most P events
                    tb = mid;
                }
                ta = tb;
                if (ta >= lo + width * (double)w)
                    ++w;
            }
        }
        window(t_end, t_end, true);
        if (lane == 0)
            s_best[0] = best_t;
        qz_sync();
        const double t = s_best[0];
        // codes (quantize_ex)
        for (uint32_t i = lane; i < P; i += 64) {
            int v = (int)fma(t, (double)s_abs[i], kQzEps);
            s_code[i] = (uint8_t)min(v, kQzCap);
        }
        qz_sync();
        if (lane == 0) {
            double ipnorm = 0.0, oxu = 0.0, cxu = 0.0;
            for (uint32_t i = 0; i < P; ++i)
                ipnorm += (s_code[i] + 0.5) * (double)s_abs[i];
            float ipnorm_inv = (float)(1.0 / ipnorm);
            if (!isnormal(ipnorm_inv))
                ipnorm_inv = 1.0f;
            const float cb = -((float)(1 << 7) - 0.5f);
            for (uint32_t i = 0; i < P; ++i) {
                const float o = s_o[i];
                const uint32_t cd = o < 0.0f ? (~(uint32_t)s_code[i]) & (uint32_t)kQzCap : s_code[i];
                const float xu = (float)(cd + (o >= 0.0f ? (1u << 7) : 0u)) + cb;
                oxu += (double)o * xu;
                cxu += (double)s_c[i] * xu;
            }
            const float l2_sqr = (float)oo;
            const float l2 = sqrtf(l2_sqr);
            float ip_resi = (float)oxu;
            const float ip_cent = (float)cxu;
            if (ip_resi == 0.0f)
                ip_resi = INFINITY;
            float *f = a.f2 + (size_t)row * 2;
            if (a.metric == 0) {
                f[0] = l2_sqr + (2.0f * l2_sqr * ip_cent / ip_resi);
                f[1] = ipnorm_inv * -2.0f * l2;
            } else {
                f[0] = 1.0f - (float)oc + (l2_sqr * ip_cent / ip_resi);
                f[1] = ipnorm_inv * -l2;
            }
        }
        for (uint32_t i = lane; i < P; i += 64) {
            const uint32_t cd = s_o[i] < 0.0f ? (~(uint32_t)s_code[i]) & (uint32_t)kQzCap : s_code[i];
            a.code[(size_t)row * P + i] = (uint8_t)cd;
        }
        qz_sync();
    }
}

struct QzBuf {
    void *p = nullptr;
    ~QzBuf() {
        if (p)
            (void)hipFree(p);
    }
};

#define QCHK(call)                                                                  \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess) {                                                     \
            set_tool_error((std::string(#call) + ": " + hipGetErrorString(e_)).c_str()); \
            return CORA_ERR_RUNTIME;                                                \
        }                                                                           \
    } while (0)

}  // namespace
}  // namespace cora

using namespace cora;

extern "C" {

int cora_tool_quantize(const float *h_x, uint64_t n, uint64_t dim, const float *h_R, uint64_t P,
                       const float *h_centroids, uint64_t nlist, const uint32_t *h_assign, int metric,
                       uint8_t *h_bits, float *h_f1, uint8_t *h_code, float *h_f2, int device) {
    if (!h_x || !h_R || !h_centroids || !h_assign || !h_bits || !h_f1 || !h_code || !h_f2 || !n || !dim ||
        P < dim || P % 64 || P > (uint64_t)kQzMaxP || !nlist || (metric != 0 && metric != 1)) {
        set_tool_error("cora_tool_quantize: invalid argument (P % 64 == 0, dim <= P <= 1024, metric 0 or 1)");
        return CORA_ERR_INVALID_ARGUMENT;
    }
    for (uint64_t i = 0; i < n; ++i)
        if (h_assign[i] >= nlist) {
            set_tool_error("cora_tool_quantize: cluster id out of range");
            return CORA_ERR_INVALID_ARGUMENT;
        }
    QCHK(hipSetDevice(device));
    const size_t chunk = std::min<size_t>(n, (size_t)1 << 20);
    QzBuf x, r, xr, c, asg, bits, f1, code, f2;
    QCHK(hipMalloc(&x.p, chunk * dim * 4));
    QCHK(hipMalloc(&r.p, dim * P * 4));
    QCHK(hipMalloc(&xr.p, chunk * P * 4));
    QCHK(hipMalloc(&c.p, nlist * P * 4));
    QCHK(hipMalloc(&asg.p, chunk * 4));
    QCHK(hipMalloc(&bits.p, chunk * P / 8));
    QCHK(hipMalloc(&f1.p, chunk * 12));
    QCHK(hipMalloc(&code.p, chunk * P));
    QCHK(hipMalloc(&f2.p, chunk * 8));
    QCHK(hipMemcpy(r.p, h_R, dim * P * 4, hipMemcpyHostToDevice));
    QCHK(hipMemcpy(c.p, h_centroids, nlist * P * 4, hipMemcpyHostToDevice));
    int cus = 256;
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    for (size_t b = 0; b < n; b += chunk) {
        const size_t rows = std::min(chunk, (size_t)n - b);
        QCHK(hipMemcpy(x.p, h_x + b * dim, rows * dim * 4, hipMemcpyHostToDevice));
        QCHK(hipMemcpy(asg.p, h_assign + b, rows * 4, hipMemcpyHostToDevice));
        launch_rotate((float *)x.p, (float *)r.p, (float *)xr.p, (uint32_t)rows, (uint32_t)dim, (uint32_t)P,
                      nullptr);
        QzArgs qa{(const float *)xr.p, (const float *)c.p, (const uint32_t *)asg.p, (uint32_t)rows,
                  (uint32_t)P, metric, (uint8_t *)bits.p, (float *)f1.p, (uint8_t *)code.p, (float *)f2.p};
        const uint32_t grid = (uint32_t)std::min<size_t>(rows, (size_t)cus * 16);
        quantize_kernel<<<grid, 64>>>(qa);
        QCHK(hipGetLastError());
        QCHK(hipMemcpy(h_bits + b * (P / 8), bits.p, rows * (P / 8), hipMemcpyDeviceToHost));
        QCHK(hipMemcpy(h_f1 + b * 3, f1.p, rows * 12, hipMemcpyDeviceToHost));
        QCHK(hipMemcpy(h_code + b * P, code.p, rows * P, hipMemcpyDeviceToHost));
        QCHK(hipMemcpy(h_f2 + b * 2, f2.p, rows * 8, hipMemcpyDeviceToHost));
    }
    return CORA_OK;
}

}  // extern "C"
