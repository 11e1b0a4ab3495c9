// Device helpers shared by the scan and vanguard translation units: wave-uniform values,
// the tile layout's code loads, the Bq=8 popcount inner product, the packed 7-bit
// ex-code inner product, ring publication and float order keys.
#pragma once

#include "engine_internal.h"

namespace cora {
namespace {

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
    return __builtin_amdgcn_readfirstlane(v);
}

__device__ __forceinline__ float uniformf(float v) {
    return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(v)));
}

__device__ __forceinline__ unsigned long long shfl0_u64(unsigned long long v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}

__device__ __forceinline__ uint32_t lane_rank(unsigned long long mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// A load through a global-memory (address space 1) pointer: a global_load, counted by
// vmcnt only. A pointer read from a kernel's parameter struct after the struct has escaped
// to an out-of-line call is generic, and its loads become flat loads, which count against
// lgkmcnt too: every wait for an LDS read then also waits for the memory loads in flight.
// HIP's vector classes are copied through a generic reference, which would turn the load
// flat again, so they are loaded as clang vectors and rebuilt.
template <class T>
__device__ __forceinline__ T gload(const void *p) {
    return *(const __attribute__((address_space(1))) T *)p;
}
template <>
__device__ __forceinline__ float4 gload<float4>(const void *p) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    const v4f v = *(const __attribute__((address_space(1))) v4f *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
template <>
__device__ __forceinline__ uint2 gload<uint2>(const void *p) {
    typedef uint32_t v2u __attribute__((ext_vector_type(2)));
    const v2u v = *(const __attribute__((address_space(1))) v2u *)p;
    return make_uint2(v.x, v.y);
}
template <>
__device__ __forceinline__ uint4 gload<uint4>(const void *p) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const v4u v = *(const __attribute__((address_space(1))) v4u *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

// W > 0: compile-time word count; W == 0: runtime word count (any P % 64 == 0, P <= 1024).
template <int W>
struct Words {
    static constexpr int kMax = W > 0 ? W : 32;
};

// Survivor stage of one wave: kCap records of 16 bytes plus their code words, about
// 4 KB, so LDS never limits the scan's occupancy below 32 waves per CU for P <= 128.
template <int W>
struct Stage {
    static constexpr int kWords = Words<W>::kMax;
    static constexpr int kFit = 4096 / (16 + 4 * kWords) / 64 * 64;
    static constexpr int kCap = kFit < 64 ? 64 : kFit;
};

template <int W>
__device__ __forceinline__ void load_codes(const uint8_t *__restrict__ tile, uint32_t lane,
                                           uint32_t rw, uint32_t (&x)[Words<W>::kMax]) {
    const uint32_t nw = W > 0 ? (uint32_t)W : rw;
    const uint4 *g4 = reinterpret_cast<const uint4 *>(tile);
#pragma unroll
    for (int g = 0; g < Words<W>::kMax / 4; ++g) {
        if ((uint32_t)(4 * g + 4) <= nw) {
            const uint4 v = g4[g * 64 + lane];
            x[4 * g] = v.x;
            x[4 * g + 1] = v.y;
            x[4 * g + 2] = v.z;
            x[4 * g + 3] = v.w;
        }
    }
    if (nw % 4 == 2) {
        const uint2 *t2 = reinterpret_cast<const uint2 *>(tile + (size_t)(nw / 4) * 1024);
        const uint2 v = t2[lane];
        x[nw - 2] = v.x;
        x[nw - 1] = v.y;
    }
}

template <int W>
__device__ __forceinline__ int popc_ip(const uint32_t (&x)[Words<W>::kMax],
                                       const uint32_t *__restrict__ planes, uint32_t rw) {
    const uint32_t nw = W > 0 ? (uint32_t)W : rw;
    int a[kBq];
#pragma unroll
    for (int j = 0; j < kBq; ++j)
        a[j] = 0;
#pragma unroll
    for (int w = 0; w < Words<W>::kMax; ++w) {
        if ((uint32_t)w < nw) {
#pragma unroll
            for (int j = 0; j < kBq; ++j)
                a[j] += __popc(x[w] & planes[j * nw + w]);
        }
    }
    int ip = -(a[kBq - 1] << (kBq - 1));
#pragma unroll
    for (int j = 0; j < kBq - 1; ++j)
        ip += a[j] << j;
    return ip;
}

// Estimator of <q',b> a scan kernel instance evaluates.
enum EstKind { kEstBitwise = 0, kEstLut4 = 1 };

// FP16 nibble-LUT <q',b> (the reference's Lut4Bit producers, filter_kernels.cuh:283-306,
// 655-708). The tile words hold dimension 32w+l at bit l; bit-reversed, they are the
// reference's words, whose nibble j (bits 31-4j..28-4j, top bit the lowest dimension)
// indexes entry [8w+j][nibble] of the query's table L [P/4][16] of FP16 values (two per u32
// word, the lower half first). Even nibbles accumulate into a0 and odd ones into a1, each
// in nibble order in FP32, and the result is a0 + a1.
template <int W>
__device__ __forceinline__ float lut4_ip(const uint32_t (&x)[Words<W>::kMax], const uint32_t *__restrict__ L,
                                         uint32_t rw) {
    const uint32_t nw = W > 0 ? (uint32_t)W : rw;
    const uint16_t *h = reinterpret_cast<const uint16_t *>(L);
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int w = 0; w < Words<W>::kMax; ++w) {
        if ((uint32_t)w < nw) {
            const uint32_t c = __builtin_bitreverse32(x[w]);
            const uint16_t *t = h + (size_t)w * 128;
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                a0 += (float)__builtin_bit_cast(_Float16, t[j * 16 + ((c >> (28 - 4 * j)) & 15u)]);
                a1 += (float)__builtin_bit_cast(_Float16, t[(j + 1) * 16 + ((c >> (24 - 4 * j)) & 15u)]);
            }
        }
    }
    return a0 + a1;
}

// LUT4 with the matrix-core kernels: how far the LUT4 lower bound of a vector can lie below
// its Bitwise lower bound (ex the Bitwise estimate, delta the query's lut_margin): |f_rescale|
// delta in exact arithmetic, plus the rounding of the two FP32 evaluations (at most 12 ulps of
// the magnitude of their terms). low_Bitwise - lut_slack < cutoff holds for every vector whose
// LUT4 lower bound is below the cutoff.
__device__ __forceinline__ float lut_slack(float delta, float fa, float fr, float fe, float gadd, float gerr,
                                           float ex, float k1) {
    return fabsf(fr) * delta +
           7.2e-7f * (fabsf(fa) + fabsf(gadd) + fabsf(fr) * (fabsf(ex) + delta + fabsf(k1)) + fabsf(fe * gerr));
}

// Two-stage <q',b>: width * ip_int rounded, then width2 * ip_res added with one rounding.
__device__ __forceinline__ float two_stage_ip(float width, int ip, float width2, int ip_res) {
    return __fmaf_rn(width2, (float)ip_res, __fmul_rn(width, (float)ip));
}

// <q', ex_code> over one 8-dimension chunk c (group g = c / 8 of 64 dimensions, k = c % 8)
// of a packed 7-bit ex-code (pack_excode.hpp:216-265) in a refinement record (rec, padded
// dimension P; engine_internal.h): per 64 dimensions, bytes 0..47 hold the low six bits of
// dimensions 0..47, and in their top two bits the bit pairs of dimensions 48..63 (bits 0-1
// in bytes 0..15, 2-3 in 16..31, 4-5 in 32..47); the u64 at bytes 48..55 holds bit 6 of
// dimension 8k+j at bit 8j+k. kL1: also accumulate sum |q'| of the chunk into *l1. Unpacked in
// 32-bit halves (four dimensions per word) so each code byte converts with one byte-to-float
// instruction.
template <bool kL1 = true>
__device__ __forceinline__ float excode_chunk_ip(const uint8_t *__restrict__ rec, uint32_t P,
                                                 const float *__restrict__ q, uint32_t c,
                                                 float *l1 = nullptr) {
    const uint32_t g = c >> 3, k = c & 7;
    const auto word = [&](uint32_t kk) {
        return *reinterpret_cast<const uint2 *>(rec + ex_record_group_word(P, g, kk));
    };
    uint32_t lo, hi;
    if (k < 6) {
        const uint2 v = word(k);
        lo = v.x & 0x3F3F3F3Fu;
        hi = v.y & 0x3F3F3F3Fu;
    } else {
        const uint32_t o = k - 6;
        const uint2 a = word(o), b = word(2 + o), d = word(4 + o);
        lo = ((a.x >> 6) & 0x03030303u) | ((b.x >> 4) & 0x0C0C0C0Cu) | ((d.x >> 2) & 0x30303030u);
        hi = ((a.y >> 6) & 0x03030303u) | ((b.y >> 4) & 0x0C0C0C0Cu) | ((d.y >> 2) & 0x30303030u);
    }
    const uint2 top = word(6);
    lo |= ((top.x >> k) & 0x01010101u) << 6;
    hi |= ((top.y >> k) & 0x01010101u) << 6;
    const float4 q0 = *reinterpret_cast<const float4 *>(q + 64 * g + 8 * k);
    const float4 q1 = *reinterpret_cast<const float4 *>(q + 64 * g + 8 * k + 4);
    float sum = 0.0f;
    sum = fmaf((float)(lo & 0xFFu), q0.x, sum);
    sum = fmaf((float)((lo >> 8) & 0xFFu), q0.y, sum);
    sum = fmaf((float)((lo >> 16) & 0xFFu), q0.z, sum);
    sum = fmaf((float)(lo >> 24), q0.w, sum);
    sum = fmaf((float)(hi & 0xFFu), q1.x, sum);
    sum = fmaf((float)((hi >> 8) & 0xFFu), q1.y, sum);
    sum = fmaf((float)((hi >> 16) & 0xFFu), q1.z, sum);
    sum = fmaf((float)(hi >> 24), q1.w, sum);
    if constexpr (kL1)
        *l1 += fabsf(q0.x) + fabsf(q0.y) + fabsf(q0.z) + fabsf(q0.w) + fabsf(q1.x) + fabsf(q1.y) +
               fabsf(q1.z) + fabsf(q1.w);
    return sum;
}

// <q', ex_code> over one whole 64-dimension group whose 56 bytes (seven 8-byte words, the
// layout above) are already in registers; q64 points at the group's 64 values of q'.
__device__ __forceinline__ float excode_group_ip(const uint2 (&grp)[7], const float *__restrict__ q64) {
    float sum = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) {
        uint32_t lo, hi;
        if (k < 6) {
            lo = grp[k].x & 0x3F3F3F3Fu;
            hi = grp[k].y & 0x3F3F3F3Fu;
        } else {
            const uint32_t o = k - 6;
            const uint2 a = grp[o], b = grp[2 + o], d = grp[4 + o];
            lo = ((a.x >> 6) & 0x03030303u) | ((b.x >> 4) & 0x0C0C0C0Cu) | ((d.x >> 2) & 0x30303030u);
            hi = ((a.y >> 6) & 0x03030303u) | ((b.y >> 4) & 0x0C0C0C0Cu) | ((d.y >> 2) & 0x30303030u);
        }
        lo |= ((grp[6].x >> k) & 0x01010101u) << 6;
        hi |= ((grp[6].y >> k) & 0x01010101u) << 6;
        const float4 q0 = *reinterpret_cast<const float4 *>(q64 + 8 * k);
        const float4 q1 = *reinterpret_cast<const float4 *>(q64 + 8 * k + 4);
        sum = fmaf((float)(lo & 0xFFu), q0.x, sum);
        sum = fmaf((float)((lo >> 8) & 0xFFu), q0.y, sum);
        sum = fmaf((float)((lo >> 16) & 0xFFu), q0.z, sum);
        sum = fmaf((float)(lo >> 24), q0.w, sum);
        sum = fmaf((float)(hi & 0xFFu), q1.x, sum);
        sum = fmaf((float)((hi >> 8) & 0xFFu), q1.y, sum);
        sum = fmaf((float)((hi >> 16) & 0xFFu), q1.z, sum);
        sum = fmaf((float)(hi >> 24), q1.w, sum);
    }
    return sum;
}


// Refined distance of a candidate (cpu_refinement.cpp:183-192) from the HBM copy of the
// ex-codes, evaluated by one lane, and its rounding bound against the CPU consumer's
// evaluation (refine_err_scale).
__device__ __forceinline__ float refine_one(const ScanParams &p, uint32_t query, uint32_t probe,
                                            uint32_t gid, float ex, float &err) {
    const uint8_t *code = p.ex_rec + (size_t)gid * p.ex_stride;
    const float *qv = p.qrot + (size_t)query * p.P;
    float ip = 0.0f, l1 = 0.0f;
    for (uint32_t c = 0; c < p.P / 8; ++c)
        ip += excode_chunk_ip(code, p.P, qv, c, &l1);
    const float2 f = *reinterpret_cast<const float2 *>(code + ex_record_factor_offset(p.P));
    const float fa = f.x, fr = f.y;
    const float gadd = p.pgadd[(size_t)query * p.nprobe + probe], kbq = p.kb[query];
    err = p.refine_err * (fabsf(fa) + fabsf(gadd) + fabsf(fr) * (128.0f * fabsf(ex) + 127.0f * l1 + fabsf(kbq)));
    return fa + gadd + fr * (128.0f * ex + ip + kbq);
}

// One 16-byte Candidate store to the host-coherent ring that writes through the GPU L2
// (system-scope coherence bits sc0 sc1). A plain store to host memory may stay in L2
// until the next system-scope release, which a producer still running never issues, so
// the CPU consumer would not see the record and the drain kernel, waiting for the CPU
// to release ring space, would never see progress.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store_ring(uint4 *slot, uint4 rec) {
    const u32x4_t v = {rec.x, rec.y, rec.z, rec.w};
    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1" ::"v"(slot), "v"(v) : "memory");
}

__device__ __noinline__ unsigned long long refresh_limit(unsigned long long *cached_limit,
                                                         int *refresh_flag,
                                                         unsigned long long *released,
                                                         unsigned long long capacity,
                                                         unsigned long long need) {
    unsigned long long lim =
        __hip_atomic_load(cached_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (lim >= need)
        return lim;
    if (atomicCAS(refresh_flag, 0, 1) == 0) {
        const unsigned long long rel =
            __hip_atomic_load(released, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
        const unsigned long long fresh = rel + capacity;
        atomicMax(cached_limit, fresh);
        __hip_atomic_store(refresh_flag, 0, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        lim = lim > fresh ? lim : fresh;
    } else {
        lim = __hip_atomic_load(cached_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return lim;
}

// Ring slot when pos is below the write limit, otherwise the HBM spill buffer; in the
// GPU-final mode, the record's own slot of the HBM array (no ring).
__device__ __forceinline__ void place_record(const QueueDev &q, unsigned long long pos,
                                             unsigned long long limit, uint4 rec) {
    if (q.final_mode) {
        if (pos < q.spill_capacity)
            q.spill[pos].item = rec;
        else
            atomicExch(q.spill_overflow, 1);
        return;
    }
    if (pos < limit) {
        store_ring(&q.items[pos & q.mask], rec);
    } else {
        const unsigned long long s = atomicAdd(q.spill_count, 1ull);
        if (s < q.spill_capacity) {
            q.spill[s].item = rec;
            q.spill[s].position = pos;
        } else {
            atomicExch(q.spill_overflow, 1);
        }
    }
}

__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_to_float(uint32_t key) {
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key);
}

}  // namespace
}  // namespace cora
