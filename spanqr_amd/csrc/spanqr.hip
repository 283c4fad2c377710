// spanqr.hip -- MI355X (gfx950) kernels and C ABI for orth(X), a robust shifted Cholesky-QR.
//
// Reference algorithm: candidates/kcholqr.py:92-112 (kcholf) with its kernels candidates/tri.py:255-412 (Gram, TRSM)
// and candidates/cuk/chol.cu:1-281 (grid-synchronised clamped Cholesky). Everything here is fp32 on gfx950 MFMA/VALU
// except the fp64 split sums and norm. The design is this project's own:
//   * every dot product is one v_mfma_f32_16x16x4_f32 chain per output element, which rounds like a sequential
//     fmaf chain in summation order, so each element has one fixed IEEE operation sequence (bit-deterministic, and
//     equal to the CPU restatement that follows the same order);
//   * the Gram is a split-K SYRK over upper 64x64 tiles with a fixed, shape-derived split count (no CU-count
//     dependence), Kahan-compensated per 32-row chunk where the reference compensates, and reduced in fp64 in split
//     order by a separate kernel that also emits fixed-order partials of ||G||_F^2;
//   * the Cholesky is one persistent kernel over 32x32 tiles synchronised by per-tile flags (no grid barriers):
//     workgroup 0 runs the diagonal chain with a two-tile-row look-ahead, each other workgroup keeps one tile row in
//     LDS; the 32x32 diagonal tiles are factored in one wavefront's registers (lane = row) and inverted (lanes
//     32-63) in the same pass, and the factor is published both row-major and packed as the solve's MFMA operands;
//   * the triangular solve is row-block parallel: for tall X a pair of wavefronts per 16 rows runs through all column
//     blocks, one 16-column half of each, with its operands streamed ahead (k_trsm_rows); otherwise each of eight
//     wavefronts owns every 8th 32-column block of a row block and applies a finished block to its later blocks with
//     MFMA (k_trsm);
//   * every kernel takes its matrix of a batch from blockIdx.z (pointer tables passed by value), so a shape group of
//     layers runs as one launch per stage.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "../../include/spanqr.h"

#pragma clang fp contract(off)

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int TB = 64;            // Gram output tile (tri.py:362 bt = 64)
constexpr int CB = 32;            // Cholesky tile, TRSM column block (chol.cu:15, tri.py:406)
constexpr int BK = 32;            // rows per Kahan chunk (tri.py:352-355)
constexpr int BUF_RSRC_WORD3 = 0x00020000;   // buffer resource word 3 for raw 32-bit loads (CDNA)
constexpr int AMAX_BLOCKS = 256;  // partial maxima written by k_amax (one per workgroup)
constexpr int TS = 33;            // row stride of 32x32 LDS tiles
constexpr uint32_t SPIN_LIMIT = 1u << 20;
// Per-matrix strides of the small per-call buffers when a plan runs a batch of same-shape matrices (blockIdx.z is
// the matrix): scalars (floats), error word and padding (uint32), Cholesky flags (uint32).
constexpr int SCAL_STRIDE = 16;
constexpr int BAR_STRIDE = 64;
constexpr int KCH_MAX_R = 1024;    // kcholf at full width: r a multiple of 32 up to this
constexpr int CH_MAXROW = KCH_MAX_R / CB;   // tiles in a tile row at most
// Cholesky flags: [nb * nb] panel flags, [nb] hand-over flags, then a call counter per Cholesky workgroup (99 at
// r = 1024, checked below)
constexpr int FLAG_STRIDE = 1280;
constexpr int CC_STRIDE = 16;      // uint32 words between the solve's column counters (one 64-byte line each)

// The caller's matrices of one launch, passed by value (a captured graph keeps the pointers): matrix z of the
// batch is p[z]. Plan-owned [K, r] buffers are passed the same way.
struct MatsIn {
    const float* p[SPANQR_MAX_BATCH];
};
struct MatsOut {
    float* p[SPANQR_MAX_BATCH];
};

// a wave-uniform address held in scalar registers (a buffer resource built from a value the compiler keeps in vector
// registers would be wrapped in a loop over its distinct values)
__device__ __forceinline__ void* uniform_ptr(const void* p) {
    const uint64_t a = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return (void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ f32x4 mfma(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float readlane(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// s = 2^-round(log2 max(m, 1e-38)) (kcholqr.py:29-30): torch's fp32 log2 (here the correctly rounded one, from a
// double log2) and round half to even; 1 for m = 0 or NaN, 0 for m = inf. mb = bits of max|x|.
__device__ float pow2_scale_bits(uint32_t mb) {
    if (mb == 0u || mb > 0x7f800000u) return 1.0f;
    if (mb == 0x7f800000u) return 0.0f;
    const float m = __uint_as_float(mb);
    const float mm = m < 1e-38f ? 1e-38f : m;
    const float y = (float)log2((double)mm);
    return ldexpf(1.0f, -(int)rintf(y));
}

// Scale from the 256 partial maxima of k_amax; every thread of a 256-thread workgroup calls it.
__device__ float block_scale(const uint32_t* __restrict__ part) {
    __shared__ uint32_t sm[4];
    uint32_t m = part[threadIdx.x];
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)m, off);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = m;
    __syncthreads();
    uint32_t t = sm[0];
    for (int i = 1; i < 4; ++i) t = sm[i] > t ? sm[i] : t;
    __syncthreads();
    return pow2_scale_bits(t);
}

// As block_scale, for a 512-thread workgroup (threads 256-511 contribute 0, the identity of the maximum of patterns)
__device__ float block_scale512(const uint32_t* __restrict__ part) {
    __shared__ uint32_t sm[8];
    uint32_t m = threadIdx.x < 256 ? part[threadIdx.x] : 0u;
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)m, off);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = m;
    __syncthreads();
    uint32_t t = sm[0];
    for (int i = 1; i < 8; ++i) t = sm[i] > t ? sm[i] : t;
    __syncthreads();
    return pow2_scale_bits(t);
}

// As block_scale, for a 128-thread workgroup (each thread takes two of the partial maxima; the maximum is exact)
__device__ float block_scale128(const uint32_t* __restrict__ part) {
    __shared__ uint32_t sm[2];
    const uint32_t a = part[threadIdx.x], b = part[threadIdx.x + 128];
    uint32_t m = a > b ? a : b;
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)m, off);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = m;
    __syncthreads();
    const uint32_t t = sm[0] > sm[1] ? sm[0] : sm[1];
    __syncthreads();
    return pow2_scale_bits(t);
}

// The 100 MHz wall clock (the s_memrealtime counter) for the instrumented Cholesky's stamps
__device__ __forceinline__ uint64_t stamp_clock() { return __builtin_amdgcn_s_memrealtime(); }

// Pivot reciprocal square root (the reference uses CUDA rsqrtf, chol.cu:45): the published fast inverse square root
// start 0x5f375a86 - (bits >> 1) (C. Lomont, "Fast Inverse Square Root", 2003) and three Newton steps
// y <- y * (1.5 - (0.5x * y) * y), each bracket one fma, so the result is a fixed function of x.
__device__ __forceinline__ float rsqrt_sw(float x) {
    float y = __uint_as_float(0x5f375a86u - (__float_as_uint(x) >> 1));
    const float h = 0.5f * x;
#pragma unroll
    for (int it = 0; it < 3; ++it) {
        float t = h * y;
        t = __builtin_fmaf(-t, y, 1.5f);
        y = y * t;
    }
    return y;
}

// ---------------------------------------------------------------------------------------------------------------
// max|x| partials (torch.linalg.vector_norm(X, inf), kcholqr.py:102): the largest bit pattern of |x| per workgroup;
// NaN patterns sort above +inf, so NaN propagates as in torch. As the first kernel of a call it also clears the
// matrix's wait-error word (bar[2], set by a bounded wait of this call's Cholesky that gave up).
// ---------------------------------------------------------------------------------------------------------------
template <int NT>
__global__ __launch_bounds__(NT) void k_amax(const MatsIn Xs, long ldx, int K, int r, uint32_t* __restrict__ part,
                                              uint32_t* bar = nullptr) {
    // the maximum is exact in any order, so the block size (and with it the order) leaves the result unchanged
    const float* __restrict__ X = Xs.p[blockIdx.z];
    part += (size_t)blockIdx.z * AMAX_BLOCKS;
    if (bar != nullptr && blockIdx.x == 0 && threadIdx.x == 0) bar[(size_t)blockIdx.z * BAR_STRIDE + 2] = 0u;
    uint32_t m = 0;
    const int r4 = r >> 2;
    const int n4 = K * r4;
    const int stride = gridDim.x * NT;
    auto amax4 = [](const float4 v) {
        const uint32_t a = __float_as_uint(v.x) & 0x7fffffffu, b = __float_as_uint(v.y) & 0x7fffffffu;
        const uint32_t c = __float_as_uint(v.z) & 0x7fffffffu, d = __float_as_uint(v.w) & 0x7fffffffu;
        const uint32_t ab = a > b ? a : b, cd = c > d ? c : d;
        return ab > cd ? ab : cd;
    };
    // four independent loads in flight per thread (one memory latency per four strides, not one per stride)
    for (int e0 = blockIdx.x * NT + threadIdx.x; e0 < n4; e0 += 4 * stride) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = e0 + u * stride;
            v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (e < n4) {
                const int row = e / r4, c4 = e - row * r4;
                v[u] = *reinterpret_cast<const float4*>(X + (size_t)row * ldx + 4 * c4);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t a = amax4(v[u]);
            m = a > m ? a : m;
        }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)m, off);
        m = o > m ? o : m;
    }
    __shared__ uint32_t sm[NT / 64];
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = sm[0];
        for (int i = 1; i < NT / 64; ++i) t = sm[i] > t ? sm[i] : t;
        part[blockIdx.x] = t;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Gram partials (tri.py:255-297, 324-375): workgroup (u, sp) computes upper 64x64 tile u = (ti, tj) of A^T A over
// rows [sp*KS, min((sp+1)*KS, K)), in 32-row chunks staged through LDS NCH at a time (rows past the split read as 0;
// the next NCH chunks are fetched into registers while these are multiplied). Eight wavefronts, each a 32x16 piece of
// the tile. KAHAN: each chunk's MFMA chain starts from 0 and is added with Kahan compensation; otherwise one chain
// runs over the whole split. SCALE: operands are s * a with the pass-1 power-of-2 scale.
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ void upper_tile(int u, int nt, int& ti, int& tj) {
    int t = 0, rem = u;
    while (rem >= nt - t) { rem -= nt - t; ++t; }
    ti = t;
    tj = t + rem;
}

// CROSS: partials of A^T B instead (the block projection of the column-blocked path, kbig.py:88-89): every tile
// u = ti * ntb + tj of the (columns of A) x (ntb * 64 columns of B) product, A's panel ti against B's panel tj.
// rc: the columns of A (rcb: of B, CROSS); when they end at a multiple of 32 but not of 64 the last tile column is
// half outside and those columns read as 0 (they only feed outputs past the bound, which are never read).
template <bool KAHAN, bool SCALE, bool CROSS = false, int NCH = 1>
__global__ __launch_bounds__(512) void k_gram(const MatsIn As, long lda, int K, int nt, int KS,
                                              const uint32_t* __restrict__ amax_part, float* __restrict__ P,
                                              const float* __restrict__ Bx = nullptr, long ldb = 0, int ntb = 0,
                                              int rc = 1 << 30, int rcb = 1 << 30) {
    const int u = blockIdx.x, sp = blockIdx.y, U = gridDim.x;
    const float* __restrict__ A = As.p[blockIdx.z];
    amax_part += (size_t)blockIdx.z * AMAX_BLOCKS;
    P += (size_t)blockIdx.z * gridDim.y * U * TB * TB;
    int ti, tj;
    if (CROSS) {
        ti = u / ntb;
        tj = u - ti * ntb;
    } else {
        upper_tile(u, nt, ti, tj);
    }
    const float* __restrict__ B = CROSS ? Bx : A;
    const long ldbb = CROSS ? ldb : lda;
    float sc = 1.0f;
    if (SCALE) sc = block_scale512(amax_part);
    __shared__ float sA[NCH * BK][TB + 16];
    __shared__ float sB[NCH * BK][TB + 16];
    // eight wavefronts: wave w computes rows 32 qi + 16 a (a = 0, 1) x columns 32 qj + 16 hb of the 64x64 tile, with
    // qi = (w >> 1) & 1, qj = w & 1, hb = w >> 2 (two per SIMD, so one's LDS traffic overlaps the other's MFMAs)
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int qi = (w >> 1) & 1, qj = w & 1, hb = w >> 2, l16 = lane & 15, lk = lane >> 4;
    f32x4 acc[2], comp[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};
        comp[a] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int k0 = sp * KS;
    const int k1 = (k0 + KS < K) ? k0 + KS : K;
    // stages of NCH BK-row chunks: stage kc + NCH BK is loaded into registers while the chunks of stage kc are
    // multiplied; rows past the split read row k1 - 1 (in bounds) and are zeroed, so the loads are unconditional
    float4 ra[NCH], rb[NCH];
    const int grow = tid >> 4, gc4 = tid & 15;   // this thread's float4 of each 32 x 64 chunk
    const bool ina = ti * TB + 4 * gc4 < rc, inb = tj * TB + 4 * gc4 < (CROSS ? rcb : rc);
    auto gload = [&](int kc) {
#pragma unroll
        for (int h = 0; h < NCH; ++h) {
            const int k = kc + h * BK + grow;
            const int kr = k < k1 ? k : k1 - 1;
            ra[h] = ina ? *reinterpret_cast<const float4*>(A + (size_t)kr * lda + ti * TB + 4 * gc4)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
            rb[h] = inb ? *reinterpret_cast<const float4*>(B + (size_t)kr * ldbb + tj * TB + 4 * gc4)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    gload(k0);
    for (int kc = k0; kc < k1; kc += NCH * BK) {
#pragma unroll
        for (int h = 0; h < NCH; ++h) {
            const bool in = kc + h * BK + grow < k1;
            float4 va = ra[h], vb = rb[h];
            if (SCALE) {
                va.x = sc * va.x; va.y = sc * va.y; va.z = sc * va.z; va.w = sc * va.w;
                vb.x = sc * vb.x; vb.y = sc * vb.y; vb.z = sc * vb.z; vb.w = sc * vb.w;
            }
            if (!in) {
                va = make_float4(0.f, 0.f, 0.f, 0.f);
                vb = make_float4(0.f, 0.f, 0.f, 0.f);
            }
            *reinterpret_cast<float4*>(&sA[h * BK + grow][4 * gc4]) = va;
            *reinterpret_cast<float4*>(&sB[h * BK + grow][4 * gc4]) = vb;
        }
        __syncthreads();
        if (kc + NCH * BK < k1) gload(kc + NCH * BK);
        __builtin_amdgcn_sched_barrier(0);   // the loads go out before the MFMAs
#pragma unroll
        for (int h = 0; h < NCH; ++h) {
            if (kc + h * BK >= k1) break;    // a chunk wholly past the split is not part of the sum
            f32x4 part[2];
#pragma unroll
            for (int a = 0; a < 2; ++a) part[a] = KAHAN ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[a];
            float xa[BK / 4], xb[BK / 4], yb[BK / 4];
#pragma unroll
            for (int kk = 0; kk < BK / 4; ++kk) {
                const int kr = h * BK + 4 * kk + lk;
                xa[kk] = sA[kr][qi * 32 + l16];
                xb[kk] = sA[kr][qi * 32 + 16 + l16];
                yb[kk] = sB[kr][qj * 32 + 16 * hb + l16];
            }
#pragma unroll
            for (int kk = 0; kk < BK / 4; ++kk) {
                part[0] = mfma(xa[kk], yb[kk], part[0]);
                part[1] = mfma(xb[kk], yb[kk], part[1]);
            }
            // issue order: the first two steps' operands, then each step's two MFMAs followed by the reads of the
            // step two ahead, so the LDS latency overlaps the chains
            __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
            for (int g = 0; g < BK / 4 - 2; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                if (KAHAN) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float y = part[a][v] - comp[a][v];
                        const float t = acc[a][v] + y;
                        comp[a][v] = (t - acc[a][v]) - y;
                        acc[a][v] = t;
                    }
                } else {
                    acc[a] = part[a];
                }
            }
        }
        __syncthreads();
    }
    float* Pt = P + ((size_t)sp * U + u) * TB * TB;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int v = 0; v < 4; ++v) Pt[(qi * 32 + a * 16 + 4 * lk + v) * TB + qj * 32 + hb * 16 + l16] = acc[a][v];
}

// ---------------------------------------------------------------------------------------------------------------
// Plain Gram partials with the operands read straight into registers: k_gram<false, false>'s partials, element for
// element, without LDS staging or barriers (taken for long splits, where it measured faster). Workgroup (u, sp) of
// four wavefronts computes upper 64x64 tile u over the split's rows, wavefront w the 32x32 block (qi, qj) =
// (w >> 1, w & 1) as four 16x16 MFMA quadrants. Lane (l16, lk) reads columns 2 l16 and 2 l16 + 1 of the block's 32
// columns of each operand strip with one 8-byte load per row 4 kk + lk of a 32-row chunk, so quadrant (a, b) holds
// the tile entries (32 qi + 2 m + a, 32 qj + 2 n + b) -- each element's chain still runs over the split's rows in
// order, four per MFMA. A buffer resource per chunk and strip whose range ends at the split's last row makes rows
// past it read as 0; a strip past the columns rc (r % 64 == 32) has an empty range. GR_DEPTH chunks are in flight
// per wavefront.
// ---------------------------------------------------------------------------------------------------------------
constexpr int GR_DEPTH = 3;   // chunks in flight per wavefront (16 loads each; vmcnt counts at most 63 outstanding)
__global__ __launch_bounds__(256) void k_gramr(const MatsIn As, long lda, int K, int nt, int KS, float* __restrict__ P,
                                               int rc) {
    const int u = blockIdx.x, sp = blockIdx.y, U = gridDim.x;
    const float* __restrict__ A = As.p[blockIdx.z];
    P += (size_t)blockIdx.z * gridDim.y * U * TB * TB;
    int ti, tj;
    upper_tile(u, nt, ti, tj);
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int qi = w >> 1, qj = w & 1, l16 = lane & 15, lk = lane >> 4;
    const int ca = ti * TB + 32 * qi, cb = tj * TB + 32 * qj;   // the block's first column in each strip
    const int k0 = sp * KS, k1 = (k0 + KS < K) ? k0 + KS : K;
    const int nch = k1 > k0 ? (k1 - k0 + BK - 1) / BK : 0;
    const char* baseA = reinterpret_cast<const char*>(A + ca);
    const char* baseB = reinterpret_cast<const char*>(A + cb);
    uint32_t off[BK / 4];   // lda < 2^24 (checked by the host): 32 rows of bytes fit 31 bits
#pragma unroll
    for (int kk = 0; kk < BK / 4; ++kk) off[kk] = ((uint32_t)(4 * kk + lk) * (uint32_t)lda + 2u * (uint32_t)l16) * 4u;
    const int last = nch > 0 ? nch - 1 : 0;
    // bytes per row of each strip's range (0: the strip is past rc and reads as 0)
    const int rowa = __builtin_amdgcn_readfirstlane(ca < rc ? (int)lda * 4 : 0);
    const int rowbb = __builtin_amdgcn_readfirstlane(cb < rc ? (int)lda * 4 : 0);
    // slot d holds chunk c with c % GR_DEPTH == d; a chunk past the split's last reads that one again (unused)
    float ra[GR_DEPTH][BK / 4][2], rb[GR_DEPTH][BK / 4][2];
    auto gload = [&](int c, float (*xa)[2], float (*xb)[2]) {
        const int kr = k0 + (c < last ? c : last) * BK;
        int nv = k1 - kr;
        nv = nv < 0 ? 0 : (nv > BK ? BK : nv);
        const int numa = __builtin_amdgcn_readfirstlane(nv * rowa);
        const int numb = __builtin_amdgcn_readfirstlane(nv * rowbb);
        const size_t rowb = (size_t)(kr < K ? kr : 0) * (size_t)lda * 4;
        const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(baseA + rowb), (short)0, numa,
                                                                            BUF_RSRC_WORD3);
        const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(baseB + rowb), (short)0, numb,
                                                                            BUF_RSRC_WORD3);
#pragma unroll
        for (int kk = 0; kk < BK / 4; ++kk) {
            const auto va = __builtin_amdgcn_raw_buffer_load_b64(rA, (int)off[kk], 0, 0);
            const auto vb = __builtin_amdgcn_raw_buffer_load_b64(rB, (int)off[kk], 0, 0);
            xa[kk][0] = __uint_as_float(va[0]);
            xa[kk][1] = __uint_as_float(va[1]);
            xb[kk][0] = __uint_as_float(vb[0]);
            xb[kk][1] = __uint_as_float(vb[1]);
        }
    };
#pragma unroll
    for (int d = 0; d < GR_DEPTH; ++d) {
        gload(d, ra[d], rb[d]);
        __builtin_amdgcn_sched_barrier(0);   // issued in slot order, so each stage waits only for its own slot
    }
    f32x4 acc[4];   // quadrant q = 2 a + b
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
    // chunk c (in slot d) into the sums; REFILL: then load chunk c + GR_DEPTH into the slot, after the MFMAs have read
    // it (the loads reuse the slot's registers: no copies, and no wait where the loop closes)
    auto stage = [&](int d, int c, bool refill) {
#pragma unroll
        for (int kk = 0; kk < BK / 4; ++kk)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[q] = mfma(ra[d][kk][q >> 1], rb[d][kk][q & 1], acc[q]);
        if (refill) gload(c + GR_DEPTH, ra[d], rb[d]);
        __builtin_amdgcn_sched_barrier(0);   // the refill goes out here, before the next chunk's MFMAs
    };
    const int nfull = nch / GR_DEPTH * GR_DEPTH;
    for (int c0 = 0; c0 < nfull; c0 += GR_DEPTH) {
#pragma unroll
        for (int d = 0; d < GR_DEPTH; ++d) stage(d, c0 + d, true);
    }
#pragma unroll
    for (int d = 0; d < GR_DEPTH - 1; ++d)
        if (nfull + d < nch) stage(d, nfull + d, false);
    // entry (32 qi + 2 (4 lk + v) + a, 32 qj + 2 l16 + b) of quadrant (a, b): quadrants (a, 0) and (a, 1) side by side
    float* Pt = P + ((size_t)sp * U + u) * TB * TB;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int i = 32 * qi + 2 * (4 * lk + v) + a, j = 32 * qj + 2 * l16;
            *reinterpret_cast<float2*>(Pt + i * TB + j) = make_float2(acc[2 * a][v], acc[2 * a + 1][v]);
        }
}

// ---------------------------------------------------------------------------------------------------------------
// Split reduction (tri.py:297/375): G = fp32(sum_s fp64(P_s)) in split order, mirrored into the lower triangle.
// MODE 0 also writes ||G||_F^2 partials: per tile u and row quad b, squares are reduced per 64-wide row by a
// shift-down tree, the four rows added in order, off-diagonal tiles doubled. MODE 1 writes D = fp32(I - G) * 0.5
// for the Newton-Schulz step (kcholqr.py:21).
// ---------------------------------------------------------------------------------------------------------------
// MODE 2 (the block projection): tile u = ti * nt + tj of a full (not symmetric) product, written once into G with
// row stride r; no norm partials.
// colcnt (MODE 0, may be null): the next Cholesky's column counters, cleared here (16 words, stride 16 per matrix).
template <int MODE>
__global__ __launch_bounds__(256) void k_reduce(const float* __restrict__ P, int S, int nt, int r,
                                                float* __restrict__ G, double* __restrict__ npart,
                                                uint32_t* colcnt = nullptr) {
    const int b = blockIdx.x, u = blockIdx.y, U = gridDim.y;
    if (MODE == 0 && colcnt != nullptr && b == 0 && u == 0 && threadIdx.x < CH_MAXROW)
        colcnt[((size_t)blockIdx.z * CH_MAXROW + threadIdx.x) * CC_STRIDE] = 0u;
    P += (size_t)blockIdx.z * S * U * TB * TB;
    G += (size_t)blockIdx.z * r * r;
    if (MODE != 2) npart += (size_t)blockIdx.z * 16 * U;
    int ti, tj;
    if (MODE == 2) {
        ti = u / nt;
        tj = u - ti * nt;
    } else {
        upper_tile(u, nt, ti, tj);
    }
    const int t = threadIdx.x, row = 4 * b + (t >> 6), col = t & 63;
    const float* p = P + (size_t)u * TB * TB + row * TB + col;
    const size_t stride = (size_t)U * TB * TB;
    // the partials in order of s, loaded eight (then four) at a time: one memory latency per batch; up to eight
    // splits in one batch (loads past S repeat partial S - 1 and are not added)
    double sum = 0.0;
    int s = 0;
    if (S <= 8) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = p[(size_t)(e < S ? e : S - 1) * stride];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (e < S) sum = sum + (double)v[e];
        s = S;
    }
    for (; s + 8 <= S; s += 8) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = p[(size_t)(s + e) * stride];
#pragma unroll
        for (int e = 0; e < 8; ++e) sum = sum + (double)v[e];
    }
    for (; s + 4 <= S; s += 4) {
        const float p0 = p[(size_t)s * stride], p1 = p[(size_t)(s + 1) * stride];
        const float p2 = p[(size_t)(s + 2) * stride], p3 = p[(size_t)(s + 3) * stride];
        sum = sum + (double)p0;
        sum = sum + (double)p1;
        sum = sum + (double)p2;
        sum = sum + (double)p3;
    }
    for (; s < S; ++s) sum = sum + (double)p[(size_t)s * stride];
    const float g = (float)sum;
    const int gi = ti * TB + row, gj = tj * TB + col;
    // a tile past r (r % 64 == 32) holds entries outside G: neither written nor counted in the norm; MODE 2's rows
    // past P's columns are written (the product has room for them, and nothing reads them), its columns past r not
    const bool in = MODE == 2 ? gj < r : (gi < r && gj < r);
    if (MODE == 0) {
        if (in) {
            G[(size_t)gi * r + gj] = g;
            if (ti != tj) G[(size_t)gj * r + gi] = g;
        }
        double q = in ? (double)g * (double)g : 0.0;
        for (int off = 32; off >= 1; off >>= 1) q = q + __shfl_down(q, off);
        __shared__ double sw[4];
        if ((t & 63) == 0) sw[t >> 6] = q;
        __syncthreads();
        if (t == 0) {
            const double tot = ((sw[0] + sw[1]) + sw[2]) + sw[3];
            npart[u * 16 + b] = (ti == tj) ? tot : 2.0 * tot;
        }
    } else if (MODE == 1) {
        const float d = ((gi == gj ? 1.0f : 0.0f) - g) * 0.5f;
        if (in) {
            G[(size_t)gi * r + gj] = d;
            if (ti != tj) G[(size_t)gj * r + gi] = d;
        }
    } else if (in) {
        G[(size_t)gi * r + gj] = g;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Gram of a short X in one launch, the split reduction inside the workgroup (tri.py:255-297, 324-375 with the sum
// over splits of tri.py:297/375): workgroup u computes the upper 32x32 tile u = (ti, tj) of G = A^T A over all K rows
// as two row splits of KS rows, one per group of four wavefronts (waves 0-3 rows [0, KS), waves 4-7 [KS, K)), each
// wavefront a 16x16 quadrant of the tile. Each wavefront reads its two 16-column operand strips of every 32-row
// chunk straight into registers in the MFMA layout, G32_DEPTH chunks ahead of the one being multiplied, and runs on
// its own (no LDS staging and no workgroup barrier until the splits are summed).
// KAHAN: each chunk's MFMA chain starts from 0 and is added with Kahan compensation; otherwise one chain runs over the
// split. SCALE: operands are s * a (the pass-1 power-of-2 scale). The splits are summed in fp64 in split order,
// rounded once, and the tile and its mirror stored in G. MODE 0 also writes the tile's ||G||_F^2 partial npart[u]
// (per quadrant, each lane's four squares added in row order and a shift-down tree over the 64 lanes; the quadrants
// (0,0), (0,1), (1,0), (1,1) added in that order; doubled off the diagonal) and clears the next Cholesky's column
// counters; MODE 1 stores D = fp32(I - G) * 0.5 for the Newton-Schulz step (kcholqr.py:21) instead of G. Per element
// the arithmetic is k_gram's + k_reduce's for the same split; only the norm partials' grouping differs. Taken where
// it measured faster than the split Gram, its reduction launch and the gap between them: short X with many tiles
// (the plan's rule).
// ---------------------------------------------------------------------------------------------------------------
constexpr int G32_DEPTH = 4; // chunks in flight per wavefront (16 loads each; vmcnt counts at most 63 outstanding)
template <bool KAHAN, bool SCALE, int MODE>
__global__ __launch_bounds__(512) void k_gram32(const MatsIn As, long lda, int K, int nb, int KS,
                                                const uint32_t* __restrict__ amax_part, float* __restrict__ G,
                                                double* __restrict__ npart, int r, uint32_t* colcnt) {
    const int u = blockIdx.x, U = gridDim.x;
    const float* __restrict__ A = As.p[blockIdx.z];
    amax_part += (size_t)blockIdx.z * AMAX_BLOCKS;
    G += (size_t)blockIdx.z * r * r;
    if (MODE == 0) npart += (size_t)blockIdx.z * U;
    if (MODE == 0 && colcnt != nullptr && u == 0 && threadIdx.x < CH_MAXROW)
        colcnt[((size_t)blockIdx.z * CH_MAXROW + threadIdx.x) * CC_STRIDE] = 0u;
    int ti, tj;
    upper_tile(u, nb, ti, tj);
    const bool diag = ti == tj;
    __shared__ float xch[4][4][64];          // split 1's accumulators, per quadrant
    __shared__ double qn[4];
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = w >> 2, q = w & 3, qi = q >> 1, qj = q & 1, l16 = lane & 15, lk = lane >> 4;
    const int k0 = g * KS, k1 = (k0 + KS < K) ? k0 + KS : K;
    const int nch = k1 > k0 ? (k1 - k0 + BK - 1) / BK : 0;       // this split's chunks
    f32x4 acc = {0.f, 0.f, 0.f, 0.f}, comp = {0.f, 0.f, 0.f, 0.f};
    // Each wavefront reads its own operands straight into the MFMA layout: lane (l16, lk) takes column 16 qi + l16 of
    // tile column ti and 16 qj + l16 of tj, rows 4 kk + lk (kk = 0..7) of each 32-row chunk, through a buffer
    // resource per chunk and strip whose range ends at the split's last row: rows past the split read as 0 without a
    // mask (the hardware's range check), and the per-lane byte offsets are the same for every chunk. Slot d holds
    // chunk c with c % G32_DEPTH == d. Loads are unconditional: a chunk past the split's last reads that one again
    // (unused; an empty split's range is empty, so nothing is read).
    float ra[G32_DEPTH][BK / 4], rb[G32_DEPTH][BK / 4];
    const char* baseA = reinterpret_cast<const char*>(A + ti * CB + 16 * qi);
    const char* baseB = reinterpret_cast<const char*>(A + tj * CB + 16 * qj);
    uint32_t off[BK / 4];   // lda < 2^24 (checked by the host): 32 rows of bytes fit 31 bits
#pragma unroll
    for (int kk = 0; kk < BK / 4; ++kk) off[kk] = ((uint32_t)(4 * kk + lk) * (uint32_t)lda + (uint32_t)l16) * 4u;
    const int last = nch > 0 ? nch - 1 : 0;
    auto gload = [&](int c, float* xa, float* xb) {
        const int kr = k0 + (c < last ? c : last) * BK;
        int nv = k1 - kr;
        nv = nv < 0 ? 0 : (nv > BK ? BK : nv);
        const int num = __builtin_amdgcn_readfirstlane(nv * (int)lda * 4);
        const size_t rowb = (size_t)(kr < K ? kr : 0) * (size_t)lda * 4;
        const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(baseA + rowb), (short)0, num,
                                                                            BUF_RSRC_WORD3);
        const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(baseB + rowb), (short)0, num,
                                                                            BUF_RSRC_WORD3);
#pragma unroll
        for (int kk = 0; kk < BK / 4; ++kk) {
            xa[kk] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rA, (int)off[kk], 0, 0));
            xb[kk] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rB, (int)off[kk], 0, 0));
        }
    };
#pragma unroll
    for (int d = 0; d < G32_DEPTH; ++d) {
        gload(d, ra[d], rb[d]);
        __builtin_amdgcn_sched_barrier(0);   // issued in slot order, so each stage waits only for its own slot
    }
    float sc = 1.0f;
    if (SCALE) sc = block_scale512(amax_part);   // (its reduction's barriers wait behind the first loads)
    // chunk c (in slot d) into the sum; REFILL: then load chunk c + G32_DEPTH into the slot, after the MFMAs have
    // read it, so the loads reuse the slot's registers (no copies, and no wait, where the loop closes)
    auto stage = [&](int d, int c, bool refill) {
        float xa[BK / 4], yb[BK / 4];
#pragma unroll
        for (int kk = 0; kk < BK / 4; ++kk) {
            xa[kk] = SCALE ? sc * ra[d][kk] : ra[d][kk];
            yb[kk] = SCALE ? sc * rb[d][kk] : rb[d][kk];
        }
        f32x4 part = KAHAN ? f32x4{0.f, 0.f, 0.f, 0.f} : acc;
#pragma unroll
        for (int kk = 0; kk < BK / 4; ++kk) part = mfma(xa[kk], yb[kk], part);
        if (refill) gload(c + G32_DEPTH, ra[d], rb[d]);
        if (KAHAN) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float y = part[v] - comp[v];
                const float t = acc[v] + y;
                comp[v] = (t - acc[v]) - y;
                acc[v] = t;
            }
        } else {
            acc = part;
        }
    };
    // whole rounds of G32_DEPTH chunks with refills (the last round's refills read chunks past the split: unused),
    // then the remaining chunks from the slots as they stand
    const int nfull = nch / G32_DEPTH * G32_DEPTH;
    for (int c0 = 0; c0 < nfull; c0 += G32_DEPTH) {
#pragma unroll
        for (int d = 0; d < G32_DEPTH; ++d) stage(d, c0 + d, true);
    }
#pragma unroll
    for (int d = 0; d < G32_DEPTH - 1; ++d)
        if (nfull + d < nch) stage(d, nfull + d, false);
    __syncthreads();
    if (g == 1)
#pragma unroll
        for (int v = 0; v < 4; ++v) xch[q][v][lane] = acc[v];
    __syncthreads();
    if (g == 0) {
        const bool two = KS < K;   // a second split exists
        float gv[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            double sum = 0.0;
            sum = sum + (double)acc[v];
            if (two) sum = sum + (double)xch[q][v][lane];
            gv[v] = (float)sum;
        }
        const int gi0 = ti * CB + 16 * qi + 4 * lk, gj = tj * CB + 16 * qj + l16;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float o = MODE == 1 ? (((gi0 + v == gj) ? 1.0f : 0.0f) - gv[v]) * 0.5f : gv[v];
            G[(size_t)(gi0 + v) * r + gj] = o;
            if (!diag) G[(size_t)gj * r + gi0 + v] = o;
        }
        if (MODE == 0) {
            double s2 = (double)gv[0] * (double)gv[0];
#pragma unroll
            for (int v = 1; v < 4; ++v) s2 = s2 + (double)gv[v] * (double)gv[v];
            for (int off = 32; off >= 1; off >>= 1) s2 = s2 + __shfl_down(s2, off);
            if (lane == 0) qn[q] = s2;
        }
    }
    if (MODE == 0) {
        __syncthreads();
        if (tid == 0) {
            const double tot = ((qn[0] + qn[1]) + qn[2]) + qn[3];
            npart[u] = diag ? tot : 2.0 * tot;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Clamped Cholesky (chol.cu:115-271): one persistent kernel over 32x32 tiles T(i, k), i >= k, nb = r / 32 tile rows,
// synchronised by per-tile flags instead of grid barriers.
//   * Workgroup 0 runs the critical chain, one step per tile row j, with T(j, j) in the registers of the wavefront
//     that factors it (wave 0 at even j, wave 7 at odd j). Step j: that wavefront factors T(j, j) and inverts the
//     factor in one pass, column pair by column pair, publishing each pair in LDS; the other of the two (the
//     look-ahead) forms the previous step's L(j+1, j-1) (Li_{j-1} is still in LDS), applies block j-1 to T(j+1, j)
//     and T(j+1, j+1), then follows the factor pair by pair: the panel L(j+1, j) by forward substitution and the
//     block j update of T(j+1, j+1), which it keeps in its registers and factors at step j+1. At the same time waves
//     1, 2, 5, 6 fetch tile row j+2 (T(j+2, j-1..j+2), handed over by its owner through column block j-2, plus the
//     owner's panel L(j+2, j-2)) while wave 3 publishes the previous step's L tiles and Li; then waves 1 and 5 form
//     the panel L(j+2, j-1), waves 2 and 6 apply the block j-2 update of T(j+2, j+1) that the owner leaves out, and
//     the four apply block j-1 to T(j+2, j), T(j+2, j+1) and the lower quadrants of T(j+2, j+2).
//   * Tile row i >= 4 is owned for the whole factorisation, in LDS, by ceil((i + 1) / OWNER_W) workgroups (parts),
//     each holding a run of its tiles. For column block j = 0..i-4 in order, a part waits for one round of flags
//     (workgroup 0's column j, and the tiles T(k, j) through block j-1 that other parts published a block ahead),
//     loads Li_j and those tiles, forms every panel it needs itself -- L(k, j) = T(k, j) Li_j^T, its own L(i, j)
//     included -- and applies T(i, k) -= L(i, j) L(k, j)^T to its tiles k = j+1..i (at the last block, j = i-4,
//     T(i, i-1) is left to workgroup 0); then it publishes T(i, j+1) through block j for the next block's
//     consumers. After block i-4 the last part hands T(i, i-3..i) to workgroup 0, two steps before workgroup 0
//     factors T(i, i).
// Every element keeps the reference order: updates by column block in increasing order, each one MFMA chain over the
// block's 32 columns. A producer publishes with an agent-scope release after its stores; a consumer polls with
// bounded waits (after `lim` polls it records an error and stops waiting, so the kernel always ends). Each
// workgroup waits only on work earlier in the (column block, panel before update) order, which with all
// workgroups resident (checked at plan creation) rules out deadlock. Flags hold the call number of the workgroup's
// own counter, so nothing is reset between calls.
// ---------------------------------------------------------------------------------------------------------------

typedef float Tile[CB][TS];

__device__ __forceinline__ void store_tile(float* dst, int ld, const Tile& src, int t = -1, int nthr = 256) {
    for (int e = (t < 0 ? (int)threadIdx.x : t); e < 256; e += nthr) {
        const int row = e >> 3, c4 = e & 7;
        float4 v;
        v.x = src[row][4 * c4 + 0]; v.y = src[row][4 * c4 + 1]; v.z = src[row][4 * c4 + 2]; v.w = src[row][4 * c4 + 3];
        *reinterpret_cast<float4*>(dst + (size_t)row * ld + 4 * c4) = v;
    }
}

// the half of store_tile_op's packed layout that holds rows 16 h .. 16 h + 15, by one wavefront
__device__ __forceinline__ void store_tile_op_half(float* dst, const Tile& src, int h, int lane) {
    for (int u = 0; u < 2; ++u) {
        const int e = 4 * (32 * u + (lane >> 1)) + 2 * h + (lane & 1);   // e & 3 = 2 h + (0 or 1): cb = h
        const int ln = e >> 2, kk0 = 4 * (e & 1), l16 = ln & 15, lk = ln >> 4;
        float4 v;
        v.x = src[16 * h + l16][4 * (kk0 + 0) + lk];
        v.y = src[16 * h + l16][4 * (kk0 + 1) + lk];
        v.z = src[16 * h + l16][4 * (kk0 + 2) + lk];
        v.w = src[16 * h + l16][4 * (kk0 + 3) + lk];
        *reinterpret_cast<float4*>(dst + 4 * e) = v;
    }
}

// rows 16 h .. 16 h + 15 of a tile, by one wavefront
__device__ __forceinline__ void store_tile_half(float* dst, int ld, const Tile& src, int h, int lane) {
    for (int e = 128 * h + lane; e < 128 * (h + 1); e += 64) {
        const int row = e >> 3, c4 = e & 7;
        float4 v;
        v.x = src[row][4 * c4 + 0]; v.y = src[row][4 * c4 + 1]; v.z = src[row][4 * c4 + 2]; v.w = src[row][4 * c4 + 3];
        *reinterpret_cast<float4*>(dst + (size_t)row * ld + 4 * c4) = v;
    }
}

// Solve operands: a factor block T (L(a, b), b < a, or Li_a for b = a) as the solve's MFMA B operands, 16 floats per
// lane, contiguous: dst[16 lane + 8 cb + kk] = T[16 cb + (lane & 15)][4 kk + (lane >> 4)], at pair index
// a (a + 1) / 2 + b of the packed factor (1024 floats per block).
__device__ __forceinline__ int op_pair(int a, int b) { return a * (a + 1) / 2 + b; }
__device__ __forceinline__ void store_tile_op(float* dst, const Tile& src, int t = -1, int nthr = 256) {
    for (int e = (t < 0 ? (int)threadIdx.x : t); e < 256; e += nthr) {
        const int lane = e >> 2, h = e & 3, cb = h >> 1, kk0 = 4 * (h & 1), l16 = lane & 15, lk = lane >> 4;
        float4 v;
        v.x = src[16 * cb + l16][4 * (kk0 + 0) + lk];
        v.y = src[16 * cb + l16][4 * (kk0 + 1) + lk];
        v.z = src[16 * cb + l16][4 * (kk0 + 2) + lk];
        v.w = src[16 * cb + l16][4 * (kk0 + 3) + lk];
        *reinterpret_cast<float4*>(dst + 4 * e) = v;
    }
}

// Up to NMAX global 32x32 tiles -> LDS tiles dst[0..n-1] by NTHR threads (thread index t): every global load is
// issued before the first LDS write, so the batch costs one memory latency. Tile q comes from srcf(q) with row
// stride ld and gets `shift` on its diagonal when (diag_mask >> q) & 1.
template <int NMAX, int NTHR, class SrcF>
__device__ __forceinline__ void load_tiles(Tile* dst, int n, int ld, uint32_t diag_mask, float shift, int t,
                                           SrcF srcf) {
    constexpr int PER = 256 / NTHR;           // float4 per thread per tile
    float4 v[NMAX][PER];
#pragma unroll
    for (int q = 0; q < NMAX; ++q)
        if (q < n)
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int e = t + u * NTHR, row = e >> 3, c4 = e & 7;
                v[q][u] = *reinterpret_cast<const float4*>(srcf(q) + (size_t)row * ld + 4 * c4);
            }
#pragma unroll
    for (int q = 0; q < NMAX; ++q)
        if (q < n)
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int e = t + u * NTHR, row = e >> 3, c4 = e & 7;
                float x[4] = {v[q][u].x, v[q][u].y, v[q][u].z, v[q][u].w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    if (((diag_mask >> q) & 1) && row == 4 * c4 + c) x[c] = x[c] + shift;
                    dst[q][row][4 * c4 + c] = x[c];
                }
            }
}

// As load_tiles without shifts, tile q from srcf(q) with row stride ldf(q) into dstf(q)
template <int NMAX, int NTHR, class DstF, class SrcF, class LdF>
__device__ __forceinline__ void load_tiles_to(int n, int t, DstF dstf, SrcF srcf, LdF ldf) {
    constexpr int PER = 256 / NTHR;
    float4 v[NMAX][PER];
#pragma unroll
    for (int q = 0; q < NMAX; ++q)
        if (q < n)
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int e = t + u * NTHR, row = e >> 3, c4 = e & 7;
                v[q][u] = *reinterpret_cast<const float4*>(srcf(q) + (size_t)row * ldf(q) + 4 * c4);
            }
#pragma unroll
    for (int q = 0; q < NMAX; ++q)
        if (q < n) {
            Tile& d = dstf(q);
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int e = t + u * NTHR, row = e >> 3, c4 = e & 7;
                d[row][4 * c4 + 0] = v[q][u].x;
                d[row][4 * c4 + 1] = v[q][u].y;
                d[row][4 * c4 + 2] = v[q][u].z;
                d[row][4 * c4 + 3] = v[q][u].w;
            }
        }
}

// the lower triangle of a diagonal tile (zeros above the diagonal), straight and transposed
__device__ __forceinline__ void store_tile_lower(float* dst, int ld, const Tile& src, bool transpose, int t, int nthr) {
    for (int e = t; e < 256; e += nthr) {
        const int row = e >> 3, c4 = e & 7;
        float x[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int col = 4 * c4 + c;
            x[c] = transpose ? ((row <= col) ? src[col][row] : 0.0f) : ((col <= row) ? src[row][col] : 0.0f);
        }
        *reinterpret_cast<float4*>(dst + (size_t)row * ld + 4 * c4) = make_float4(x[0], x[1], x[2], x[3]);
    }
}

// The four-quadrant tile helpers below are called by every wavefront of the workgroup (they contain workgroup
// barriers); the work is done by waves 0-3 (one 16x16 quadrant each) when `on` is set, the others only pass the
// barriers.

// One wave's quadrant (bi, bj) of NT tiles tf(t0), tf(t0 + 2), ...: acc[u] = A_u Li^T over the chain m < 4 NK
// (NK = 4 (bj + 1)), every operand read first, the NT independent chains interleaved
template <int NT, int NK, class TF>
__device__ __forceinline__ void panel_chains(TF tf, int t0, const float (&bv)[8], f32x4 (&acc)[4], int bi, int l16,
                                             int lk) {
    float a[NT][NK];
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) a[u][kk] = tf(t0 + 2 * u)[16 * bi + l16][4 * kk + lk];
#pragma unroll
    for (int u = 0; u < NT; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
        for (int u = 0; u < NT; ++u) acc[u] = mfma(a[u][kk], bv[kk], acc[u]);
}

// In place, n tiles tf(q) = tf(q) Li^T, each element a chain over m < 16 (bj + 1) from +0 (Li is lower triangular,
// chol.cu panel), by the eight wavefronts in chunks of up to eight tiles: wave w takes quadrant (bi, bj) = (w & 3) of
// the chunk's tiles w >> 2, (w >> 2) + 2, ...; every wave reads its operands and runs its chains, then, after a
// workgroup barrier, writes the results.
template <class TF>
__device__ __forceinline__ void panels_inplace(int n, TF tf, const Tile& li) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, l16 = lane & 15,
              lk = lane >> 4, qd = w & 3, bi = qd >> 1, bj = qd & 1, half = w >> 2;
    float bv[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) bv[kk] = li[16 * bj + l16][4 * kk + lk];   // (bj = 0 uses kk < 4)
    for (int c0 = 0; c0 < n; c0 += 8) {
        const int nc = n - c0 < 8 ? n - c0 : 8;
        const int nt = (nc - half + 1) / 2;
        auto tfc = [&](int t) -> Tile& { return tf(c0 + t); };
        f32x4 acc[4];
        if (bj == 0) {
            switch (nt) {
                case 1: panel_chains<1, 4>(tfc, half, bv, acc, bi, l16, lk); break;
                case 2: panel_chains<2, 4>(tfc, half, bv, acc, bi, l16, lk); break;
                case 3: panel_chains<3, 4>(tfc, half, bv, acc, bi, l16, lk); break;
                case 4: panel_chains<4, 4>(tfc, half, bv, acc, bi, l16, lk); break;
                default: break;
            }
        } else {
            switch (nt) {
                case 1: panel_chains<1, 8>(tfc, half, bv, acc, bi, l16, lk); break;
                case 2: panel_chains<2, 8>(tfc, half, bv, acc, bi, l16, lk); break;
                case 3: panel_chains<3, 8>(tfc, half, bv, acc, bi, l16, lk); break;
                case 4: panel_chains<4, 8>(tfc, half, bv, acc, bi, l16, lk); break;
                default: break;
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (u < nt) {
                Tile& t = tfc(half + 2 * u);
#pragma unroll
                for (int v = 0; v < 4; ++v) t[16 * bi + 4 * lk + v][16 * bj + l16] = acc[u][v];
            }
        __syncthreads();
    }
}

// quadrant masks: the row half h of the A operand (bi = h) and the row half of the B operand (bj = h) that a set of
// 16x16 quadrants qd = 2 bi + bj uses
constexpr bool qm_uses_a(int qm, int h) { return (qm >> (2 * h)) & 3; }
constexpr bool qm_uses_b(int qm, int h) { return (qm >> h) & 5; }

// One wave: out = in Li^T on the quadrants whose bit is set in QM (all four: a whole 32x32 tile; out must not alias
// in). Each operand element is read from LDS once and the quadrants' MFMA chains (over m < 16 (bj + 1)) interleaved.
template <int QM = 0xF>
__device__ __forceinline__ void panel32_wave(Tile& out, const Tile& in, const Tile& li) {
    const int lane = threadIdx.x & 63, l16 = lane & 15, lk = lane >> 4;
    float a[2][8], b[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            a[h][kk] = qm_uses_a(QM, h) ? in[16 * h + l16][4 * kk + lk] : 0.0f;
            b[h][kk] = (qm_uses_b(QM, h) && kk < 4 * (h + 1)) ? li[16 * h + l16][4 * kk + lk] : 0.0f;
        }
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const int bi = qd >> 1, bj = qd & 1;
            if (((QM >> qd) & 1) && kk < 4 * (bj + 1)) acc[qd] = mfma(a[bi][kk], b[bj][kk], acc[qd]);
        }
#pragma unroll
    for (int qd = 0; qd < 4; ++qd)
        if ((QM >> qd) & 1)
#pragma unroll
            for (int v = 0; v < 4; ++v) out[16 * (qd >> 1) + 4 * lk + v][16 * (qd & 1) + l16] = acc[qd][v];
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the tile is written before this wave reads it back
    __builtin_amdgcn_wave_barrier();
}

// One wave: dst = C - Pi Pk^T on the 16x16 quadrants qd = 2 bi + bj whose bit is set in QM (dst may alias C);
// the operands those quadrants use read once, their chains (over m = 0..31 from C) interleaved.
template <int QM>
__device__ __forceinline__ void update32_wave_q(Tile& dst, const Tile& C, const Tile& Pi, const Tile& Pk) {
    const int lane = threadIdx.x & 63, l16 = lane & 15, lk = lane >> 4;
    float a[2][8], b[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            a[h][kk] = qm_uses_a(QM, h) ? -Pi[16 * h + l16][4 * kk + lk] : 0.0f;
            b[h][kk] = qm_uses_b(QM, h) ? Pk[16 * h + l16][4 * kk + lk] : 0.0f;
        }
    f32x4 acc[4];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd)
#pragma unroll
        for (int v = 0; v < 4; ++v)
            acc[qd][v] = ((QM >> qd) & 1) ? C[16 * (qd >> 1) + 4 * lk + v][16 * (qd & 1) + l16] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd)
            if ((QM >> qd) & 1) acc[qd] = mfma(a[qd >> 1][kk], b[qd & 1][kk], acc[qd]);
#pragma unroll
    for (int qd = 0; qd < 4; ++qd)
        if ((QM >> qd) & 1)
#pragma unroll
            for (int v = 0; v < 4; ++v) dst[16 * (qd >> 1) + 4 * lk + v][16 * (qd & 1) + l16] = acc[qd][v];
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
}

// whole tile (LOWER: without the upper 16x16 block), in place or to dst
template <bool LOWER>
__device__ __forceinline__ void update32_wave_to(Tile& dst, const Tile& C, const Tile& Pi, const Tile& Pk) {
    update32_wave_q<LOWER ? 0xD : 0xF>(dst, C, Pi, Pk);
}
template <bool LOWER>
__device__ __forceinline__ void update32_wave(Tile& C, const Tile& Pi, const Tile& Pk) {
    update32_wave_q<LOWER ? 0xD : 0xF>(C, C, Pi, Pk);
}

// Poll an agent-scope flag until it holds `ep` (bounded), then acquire. Called by one lane.
__device__ __forceinline__ void wait_flag(const uint32_t* f, uint32_t ep, uint32_t* err, bool& dead,
                                          uint32_t lim = SPIN_LIMIT) {
    uint32_t n = 0;
    while (!dead && __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != ep) {
        if (++n > lim) {
            __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            dead = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Poll up to 64 agent-scope flags at once, each lane watching its own (`mine`; nullptr: nothing to wait for), until
// all hold `ep` (bounded), then acquire. Called by a whole wavefront; costs one round trip after the last publication
// instead of one per flag.
__device__ __forceinline__ void wait_flags_wave(const uint32_t* mine, uint32_t ep, uint32_t* err, bool& dead,
                                                uint32_t lim) {
    const int lane = threadIdx.x & 63;
    uint32_t polls = 0;
    while (!dead) {
        const bool ok = mine == nullptr || __hip_atomic_load(mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ep;
        if (__all(ok)) break;
        if (++polls > lim) {
            if (lane == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            dead = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Publish: the calling lane's wave (or, after a workgroup sync, the workgroup) has its stores issued. release()
// waits for them and makes them visible at agent scope (one L2 write-back); the flags that follow are plain
// agent-scope stores. The fence's write-back (buffer_wbl2) is counted in vmcnt, and the wait for it must come
// before the flag store: the compiler drops its own wait where no other vector memory operation is outstanding,
// and a flag that overtakes the write-back lets a reader on another XCD fetch the previous launch's data from
// memory. The explicit wait keeps the order.
__device__ __forceinline__ void release() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the L2 write-back has completed
}
__device__ __forceinline__ void set_flag(uint32_t* f, uint32_t ep) {
    __hip_atomic_store(f, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_flag(uint32_t* f, uint32_t ep) {
    release();
    set_flag(f, ep);
}

// Barrier of some waves of a workgroup while the others keep running: an LDS counter that each participating
// wave's lane 0 bumps after its own LDS writes have completed, then waits for (bounded) until it reaches `target`
// (the number of participants times the number of times this barrier has been passed).
__device__ __forceinline__ void wave_group_barrier(uint32_t* ctr, uint32_t target, uint32_t* err, bool& dead,
                                                   uint32_t lim) {
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    if ((threadIdx.x & 63) == 0) {
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        uint32_t n = 0;
        while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
            if (++n > lim) {
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                dead = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __builtin_amdgcn_wave_barrier();
}

// Wait (lane 0 polls, bounded) until an LDS word that another wavefront of the workgroup raises reaches `target`.
__device__ __forceinline__ void wait_lds(const uint32_t* word, uint32_t target, uint32_t* err, bool& dead,
                                         uint32_t lim) {
    if ((threadIdx.x & 63) == 0) {
        uint32_t n = 0;
        while (!dead && __hip_atomic_load(word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
            if (++n > lim) {
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                dead = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __builtin_amdgcn_wave_barrier();
}

typedef float f32x16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// The v_mfma_f32_32x32x2_f32 accumulator layout of a 32x32 tile: lane l, register v holds element (m, n) with
// m = 8 (v >> 2) + 4 (l >> 5) + (v & 3), n = l & 31. A symmetric tile loaded from its lower triangle, and a tile's
// transpose:
__device__ __forceinline__ void load_sym(f32x16& C, const Tile& T) {
    const int lane = threadIdx.x & 63, h = lane >> 5, n = lane & 31;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int m = 8 * (v >> 2) + 4 * h + (v & 3);
        C[v] = m >= n ? T[m][n] : T[n][m];
    }
}
__device__ __forceinline__ void load_tr(f32x16& C, const Tile& T) {
    const int lane = threadIdx.x & 63, h = lane >> 5, n = lane & 31;
#pragma unroll
    for (int v = 0; v < 16; ++v) C[v] = T[n][8 * (v >> 2) + 4 * h + (v & 3)];
}

// Tile factor of diagonal step j (chol.cu:131-168), every trailing update on the matrix cores, by one wavefront. C
// holds T(j, j) through block j-1 in the accumulator layout (kept whole and symmetric: element (m, n) and (n, m)
// receive the same operations, so row c -- register v(c) = 4 (c >> 3) + (c & 3) on the lanes of half (c >> 2) & 1 --
// is also column c). Columns go in pairs (c, c+1): pivot c from the diagonal element (piv = fmaxf(d, tau),
// q = rsqrt(piv); a NaN pivot becomes tau), L's column c = row c times q; the second pivot from scalars
// (s = L(c+1, c), d' = fma(-s, s, C(c+1, c+1)), the operations that give lane c+1 of a per-row factor its own
// values), row c+1 takes column c's update on the VALU; the two columns become one MFMA operand (lanes 0-31 column c,
// 32-63 column c+1: one cross-half swap) and a single 32x32x2 MFMA applies both columns to the whole tile, k = c then
// c+1: every element receives its updates in column order (an MFMA rounds each k step like a sequential fmaf). The
// inverse's accumulator W (from the identity) takes the same column pairs against its rows X_c = W_c q_c (W_{c+1}
// first updated by X_c): the forward substitution x = (delta - sum_m L_im x_m) q_i, column by column. Elements of
// finished rows and columns take further updates that nothing reads. Outputs: L(j, j) to dl (upper triangle
// unspecified, diagonal piv q patched in at the end), the inverse to Li and to gli (row stride 32), pq[c] = piv q;
// per pair p, for the wavefront that forms the panel below (row_pairs): L's two columns in dl, fq[4p..4p+2] =
// q_c, q_{c+1}, L(c+1, c), and then the LDS word fcnt = base + p + 1 (a plain store after them: one wavefront's LDS
// operations complete in issue order). Global stores are left in flight.
__device__ __forceinline__ void factor_pairs(f32x16& C, float* pq, float* fq, uint32_t* fcnt, uint32_t base, float tau,
                                             Tile& dl, Tile& Li, float* gli) {
    const int lane = threadIdx.x & 63, h = lane >> 5, n = lane & 31;
    f32x16 W;
#pragma unroll
    for (int v = 0; v < 16; ++v) W[v] = (8 * (v >> 2) + 4 * h + (v & 3)) == n ? 1.0f : 0.0f;
#pragma unroll
    for (int p = 0; p < CB / 2; ++p) {
        const int c = 2 * p;
        const int v0 = 4 * (c >> 3) + (c & 3), hh = (c >> 2) & 1, lc = c + 32 * hh;   // row c: register, half, lane
        const bool mine = h == hh;
        const float x = readlane(C[v0], lc + 1), y = readlane(C[v0 + 1], lc + 1);
        const float pn0 = fmaxf(readlane(C[v0], lc), tau);
        const float q0 = rsqrt_sw(pn0);
        const float s = x * q0;                          // L(c+1, c)
        const float pn1 = fmaxf(__builtin_fmaf(-s, s, y), tau);
        const float q1 = rsqrt_sw(pn1);
        const float Lc = C[v0] * q0;
        const float cu = __builtin_fmaf(-Lc, s, C[v0 + 1]);   // row c+1 by column c (lanes of half hh only: the
        C[v0 + 1] = mine ? cu : C[v0 + 1];                    // other half of the register holds another row)
        const float Lc1 = C[v0 + 1] * q1;
        const auto la = __builtin_amdgcn_permlane32_swap(__float_as_uint(Lc), __float_as_uint(Lc1), false, false);
        const float a = __uint_as_float(hh == 0 ? la[0] : la[1]);    // lane l: L(l & 31, c + (l >> 5))
        C = mfma32(-a, a, C);
        const float Xc = W[v0] * q0;
        const float wu = __builtin_fmaf(-Xc, s, W[v0 + 1]);
        W[v0 + 1] = mine ? wu : W[v0 + 1];
        const float Xc1 = W[v0 + 1] * q1;
        const auto lx = __builtin_amdgcn_permlane32_swap(__float_as_uint(Xc), __float_as_uint(Xc1), false, false);
        const float bx = __uint_as_float(hh == 0 ? lx[0] : lx[1]);   // lane l: X(c + (l >> 5), l & 31)
        W = mfma32(-a, bx, W);
        dl[n][c + h] = a;
        Li[c + h][n] = bx;
        gli[(c + h) * CB + n] = bx;
        if (lane == 0) {
            pq[c] = pn0 * q0;
            pq[c + 1] = pn1 * q1;
            fq[4 * p] = q0;
            fq[4 * p + 1] = q1;
            fq[4 * p + 2] = s;
            asm volatile("" ::: "memory");
            __hip_atomic_store(fcnt, base + p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    if (lane < CB) dl[lane][lane] = pq[lane];
    __builtin_amdgcn_wave_barrier();
}

// The look-ahead of step j on tile row j+1, by a second wavefront: C = T(j+1, j+1) and T2 = the transpose of
// T(j+1, j) through block j-1 from the tiles Dt = T(j+1, j+1) (lower triangle) and Xt = T(j+1, j) through block
// j-2 and the panels P2 = L(j+1, j-1), P1 = L(j, j-1) (chol.cu:182-271's trailing update, each element an fmaf
// chain over the 32 columns in order: C(m, n) -= P2(m, c) P2(n, c), T2(m, n) -= P1(m, c) P2(n, c), two columns per
// 32x32x2 MFMA).
__device__ __forceinline__ void row_setup(f32x16& C, f32x16& T2, const Tile& Dt, const Tile& Xt, const Tile& P2,
                                          const Tile& P1) {
    const int lane = threadIdx.x & 63, h = lane >> 5, n = lane & 31;
    load_sym(C, Dt);
    load_tr(T2, Xt);
#pragma unroll
    for (int k = 0; k < CB / 2; ++k) {
        const float v2 = P2[n][2 * k + h], v1 = P1[n][2 * k + h];
        C = mfma32(-v2, v2, C);
        T2 = mfma32(-v1, v2, T2);
    }
}

// Then the panel L(j+1, j) by forward substitution beside the tile factor (row c of T2 times q_c after the updates
// by columns < c: the pair's first column on the VALU, then both by one MFMA against L's column pair), and C takes
// the panel's column pairs -- the look-ahead update T(j+1, j+1) -= L(j+1, j) L(j+1, j)^T -- so that on return C holds
// T(j+1, j+1) through block j, the next step's tile. Pair k's operands are read one pair ahead together with the
// factor's word fcnt (read first: the factor stores a pair's operands before raising fcnt to base + k + 1, and one
// wavefront's LDS operations complete in issue order); if that word shows them not yet there, the wavefront polls
// (bounded) and reads them again. Outputs: L(j+1, j) to P1 and to gP1 (row stride ldg); global stores are left in
// flight.
__device__ __forceinline__ void row_pairs(f32x16& C, f32x16& T2, const float* fq, const uint32_t* fcnt, uint32_t base,
                                          const Tile& dl, Tile& P1, float* gP1, long ldg, uint32_t* err, bool& dead,
                                          uint32_t lim) {
    const int lane = threadIdx.x & 63, h = lane >> 5, n = lane & 31;
    uint32_t polls = 0;
    uint32_t got;
    float an;
    float4 fn;
    auto fetch = [&](int k) {
        got = __hip_atomic_load(fcnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        asm volatile("" ::: "memory");
        an = dl[n][2 * k + h];
        fn = *reinterpret_cast<const float4*>(fq + 4 * k);
    };
    fetch(0);
#pragma unroll
    for (int k = 0; k < CB / 2; ++k) {
        const int c = 2 * k, v0 = 4 * (c >> 3) + (c & 3), hh = (c >> 2) & 1;
        const bool mine = h == hh;
        if ((uint32_t)__builtin_amdgcn_readfirstlane(got) < base + k + 1) {
            while (!dead && (uint32_t)__builtin_amdgcn_readfirstlane(__hip_atomic_load(fcnt, __ATOMIC_ACQUIRE,
                                                                                       __HIP_MEMORY_SCOPE_WORKGROUP)) <
                                base + k + 1) {
                if (++polls > lim) {
                    if (lane == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    dead = true;
                }
            }
            fetch(k);
        }
        const float a = an;                              // lane l: L(l & 31, c + (l >> 5))
        const float q0 = fn.x, q1 = fn.y, s = fn.z;
        if (k + 1 < CB / 2) fetch(k + 1);
        const float l0 = T2[v0] * q0;
        const float tu = __builtin_fmaf(-l0, s, T2[v0 + 1]);
        T2[v0 + 1] = mine ? tu : T2[v0 + 1];
        const float l1 = T2[v0 + 1] * q1;
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l0), __float_as_uint(l1), false, false);
        const float b2 = __uint_as_float(hh == 0 ? sw[0] : sw[1]);   // lane l: L(j+1, j)(l & 31, c + (l >> 5))
        T2 = mfma32(-a, b2, T2);
        C = mfma32(-b2, b2, C);
        P1[n][c + h] = b2;
        gP1[(size_t)n * ldg + c + h] = b2;
    }
}

constexpr int CH_WG0_TILES = 23;   // workgroup 0: D[2], X1, R2[2][5], dl[2], li[2], P1[2], P2[2], C2[2]
// Owner parts: tile row i (i + 1 tiles) is split over P = ceil((i + 1) / w) workgroups, each holding a run of
// consecutive tiles T(i, s..e-1): widths floor((i + 1) / P), the last (i + 1) % P parts one wider, so that for
// w >= 6 the last part (which holds T(i, i-3..i) and hands them to workgroup 0) has at least 4 tiles for every row
// i >= 4. A part's work per column block shrinks with its width, so long rows keep up with workgroup 0's steps; the
// plan picks w (a single matrix: OWNER_W; a batch: wider parts where that puts it in fewer co-resident launches).
constexpr int OWNER_W = 6;       // (6: the best of 6, 7, 8 and 16 at r = 512 and of 6, 8 and 16 at r = 256)
constexpr int OWNER_WMAX = 16;   // widest parts (one part per row up to r = 512)
__host__ __device__ constexpr int row_parts(int i, int w) { return (i + w) / w; }
__host__ __device__ inline void part_range(int i, int q, int w, int& s, int& e) {
    const int n = i + 1, P = row_parts(i, w), base = n / P, lo = P - n % P;   // parts q < lo have base tiles
    s = q * base + (q > lo ? q - lo : 0);
    e = s + base + (q >= lo ? 1 : 0);
}
// workgroup b >= 1 of the Cholesky: row i, tiles [s, e); the rows' parts in order of i, then of s
__device__ inline void owner_part(int b, int nb, int w, int& i, int& s, int& e) {
    int q = b - 1;
    i = 4;
    while (i < nb - 1 && q >= row_parts(i, w)) {
        q -= row_parts(i, w);
        ++i;
    }
    part_range(i, q, w, s, e);
}
// LDS tiles of an owner part: its row tiles and their panels (at most min(nb, w) each), Li_j and L(i, j)
__host__ __device__ constexpr int owner_lds_tiles(int nb, int w) { return 2 * (nb < w ? nb : w) + 2; }
// workgroups of one Cholesky: workgroup 0 and the parts of rows 4..nb-1
constexpr int chol_workgroups(int nb, int w) {
    int n = 1;
    for (int i = 4; i < nb; ++i) n += row_parts(i, w);
    return n;
}

struct CholWG0 {
    Tile D[2];      // D[j & 1]: T(j, j) through block j-1 (factored at step j); D[(j+1) & 1]: T(j+1, j+1)
    Tile X1;        // T(j+1, j) through block j-1 (its panel is L(j+1, j)); D[0], D[1], X1 are loaded as one batch
    Tile R2[2][5];  // R2[j & 1]: tile row j+2: T(j+2, j-1..j+2) as handed over (through block j-2), then through
                    // block j-1; [4] = L(j+2, j-2): the owner's last panel of row j+2. Read again at step j+1.
    Tile dl[2];     // L(j, j)
    Tile li[2];     // Li_j
    Tile P1[2];     // L(j+1, j)
    Tile P2[2];     // L(j+2, j)
    Tile C2[2];     // L(j+2, j-1) (the catch-up panel of row j+2)
};
static_assert(sizeof(CholWG0) == CH_WG0_TILES * sizeof(Tile), "workgroup 0's tiles");

size_t chol_lds_bytes(int r, int w) {
    const int owner_tiles = owner_lds_tiles(r / CB, w);
    const int tiles = owner_tiles > CH_WG0_TILES ? owner_tiles : CH_WG0_TILES;
    return (size_t)tiles * sizeof(Tile) + 256 * sizeof(float);
}

// nb = r/32 tile rows; grid = chol_workgroups(nb) workgroups. With nnp == 0 the shift is 0 and tau_rel is the absolute
// pivot floor (chol32's contract); otherwise ||G||_F comes from the nnp fp64 partials: lane l of wave 0 sums
// npart[l], npart[l + 64], ... in order, then a shift-down tree over the 64 lane sums; nrm = sqrtf(fp32(sum)),
// shift = alpha * nrm added to the diagonal after the first load, tau = tau_rel * nrm + 1e-30 (kcholqr.py:107-109).
// flags: [nb * nb] panel flags (L(i, j) published; (j, j): L(j, j) and Li_j), [nb] hand-over flags (tile row i),
// [64] per-workgroup call counters. STAMP: workgroup 0 records the wall clock at 1 + 4j + s for step j: s = 0 step
// start, 1 step end, 2 look-ahead done, 3 tile factor done; slot 0 is the kernel start, 1 + 4 nb the end;
// 2 + 4 nb + j: wave 1's row work of step j done; 2 + 5 nb + j: wave 3's done; 2 + 6 nb + j: the hand-over of row j+2
// seen; 2 + 7 nb + j: row j+2 fetched; 2 + 8 nb + j: its panel L(j+2, j-1) formed; 2 + 9 nb + j: wave 2 done;
// 2 + 10 nb + 6 i + s: the owner of row i's last part at its last block: s = 0 flags seen, 1 operands loaded,
// 2 panels formed, 3 row handed over, 4 update done, 5 hand-over stores done; 2 + 16 nb + 8 j + s: the last row's
// last part at block j: s = 0 flags seen, 1 operands loaded, 2 panels formed, 3 block done, 4 T(i, j+1) published.
// Workgroups of eight wavefronts (workgroup 0: waves 0 and 7 the tile factor and the look-ahead in turn, waves 1, 2,
// 5, 6 the row of step j+2, wave 3 the publication, wave 4 the early write-back; owners: all eight on the panels
// and the row update, two wavefronts per SIMD so that one's LDS traffic overlaps the other's MFMA chain).
// Flags: (j, j) workgroup 0's column j (L(j, j), Li_j, L(j+1, j), T(j+2, j)); (i, j), i > j, the tile T(i, j)
// through block j-1 in its slot of A (an owner part, a block ahead); hand-over flag i, T(i, i-3..i) through block
// i-4 (the last part of row i).
// colcnt (may be null): per column block k, a counter (stride CC_STRIDE) that every producer of the packed operands
// of column k (Li_k and L(i, k), i > k) raises once those are released, for the solve that runs in the same launch:
// the owner part holding T(i, j) credits column j at the release that ends block j (the last part's hand-over
// release at its last block); workgroup 0 credits
// column k at the release that opens step k+2 (its stores of column k's operands completed during step k+1), column
// nb-2 at a release of its own in the last step, and column nb-1 (Li_{nb-1} alone) right after the last tile factor.
// Column k is complete at 1 + max(0, nb - 4 - k) credits; the counters start at zero.
static_assert(chol_workgroups(CH_MAXROW, OWNER_W) <= FLAG_STRIDE - CH_MAXROW * (CH_MAXROW + 1),
              "a call counter per Cholesky workgroup after the panel and hand-over flags");

__device__ __forceinline__ void credit(uint32_t* colcnt, int k) {
    if (colcnt != nullptr) __hip_atomic_fetch_add(colcnt + (size_t)k * CC_STRIDE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The Cholesky of workgroup b of matrix z (the pointers address matrix 0 of the launch).
template <bool STAMP>
__device__ __forceinline__ void chol_body(const int b, const size_t z, float* A, int r, const double* __restrict__ npart,
                                          int nnp, float alpha, float tau_rel, float* L, float* Li, float* Lp,
                                          uint32_t* bar, uint32_t* flags, float* scal, uint64_t* stamps, uint32_t lim,
                                          uint32_t* colcnt, int ow, const float* tau_ptr = nullptr) {
    extern __shared__ float4 chol_lds[];
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int nb = r / CB;
    {
        A += z * r * r;
        L += z * r * r;
        Li += z * r * CB;
        Lp += z * (nb * (nb + 1) / 2) * CB * CB;
        npart += z * nnp;
        bar += z * BAR_STRIDE;
        flags += z * FLAG_STRIDE;
        if (scal != nullptr) scal += z * SCAL_STRIDE;
        if (colcnt != nullptr) colcnt += z * CC_STRIDE * CH_MAXROW;
    }
    uint32_t* err = bar + 2;
    uint32_t* flagL = flags;
    uint32_t* flagT = flags + nb * nb;
    uint32_t* cnt = flags + nb * nb + nb;
    bool dead = false;
    if (STAMP && b == 0 && tid == 0) stamps[0] = stamp_clock();
    const uint32_t ep = cnt[b] + 1;        // this call's number (every workgroup runs every call)
    // misc: [0..2] nrm, shift, tau; workgroup 0's LDS words: [4] the row wavefronts' barrier counter, [5] the last step
    // whose L(j+2, j) is formed, [6] the halves of L(j+2, j-1) formed, [7] the tile factor's pairs done; [32..63] the tile factor's diagonal (piv q),
    // [64..127] its per-pair scalars
    float* misc = reinterpret_cast<float*>(chol_lds);
    Tile* tiles = reinterpret_cast<Tile*>(misc + 256);
    // an owner part: tile row oi, tiles T(oi, os..oe-1)
    int oi = 0, os = 0, oe = 0;
    if (b > 0) owner_part(b, nb, ow, oi, os, oe);
    // Waves 1-2 load the workgroup's first tiles (workgroup 0: T(0, 0), T(1, 1), T(1, 0) into D[0], D[1], X1; an
    // owner part: its tiles of the row) while wave 0 sums the norm partials; the diagonal shift is added once it is
    // known (the same single addition as on a shifted load).
    if (w == 1 || w == 2) {
        if (b == 0) {
            load_tiles<3, 128>(tiles, nb > 1 ? 3 : 1, r, 0u, 0.f, tid - 64, [&](int q) {
                return A + (q == 0 ? (size_t)0 : (size_t)CB * r + (q == 1 ? CB : 0));
            });
        } else {
            load_tiles<OWNER_WMAX, 128>(tiles, oe - os, r, 0u, 0.f, tid - 64,
                                     [&](int q) { return A + (size_t)CB * oi * r + (size_t)CB * (os + q); });
        }
    }
    if (w == 0) {
        // lane sums in index order, the partials loaded eight at a time (one memory latency per eight)
        double s = 0.0;
        for (int p0 = lane; p0 < nnp; p0 += 8 * 64) {
            double v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = (p0 + 64 * u < nnp) ? npart[p0 + 64 * u] : 0.0;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (p0 + 64 * u < nnp) s = s + v[u];
        }
        for (int off = 32; off >= 1; off >>= 1) s = s + __shfl_down(s, off);
        if (lane == 0) {
            reinterpret_cast<uint32_t*>(misc)[4] = 0u;
            reinterpret_cast<uint32_t*>(misc)[5] = 0u;
            reinterpret_cast<uint32_t*>(misc)[6] = 0u;
            reinterpret_cast<uint32_t*>(misc)[7] = 0u;
            if (nnp > 0) {
                const float nrm = sqrtf((float)s);
                misc[0] = nrm;
                misc[1] = alpha * nrm;
                misc[2] = tau_rel * nrm + 1e-30f;
            } else {
                misc[0] = 0.0f;
                misc[1] = 0.0f;
                misc[2] = tau_ptr != nullptr ? *tau_ptr : tau_rel;
            }
        }
    }
    __syncthreads();
    const float shift = misc[1], tau = misc[2];
    if (tid < CB) {
        if (b == 0) {
            tiles[0][tid][tid] = tiles[0][tid][tid] + shift;
            if (nb > 1) tiles[1][tid][tid] = tiles[1][tid][tid] + shift;
        } else if (oe == oi + 1) {
            tiles[oi - os][tid][tid] = tiles[oi - os][tid][tid] + shift;
        }
    }
    __syncthreads();
    float* pq = misc + 32;

    if (b == 0) {
        if (tid == 0 && scal != nullptr) {
            scal[0] = misc[0];
            scal[1] = tau;
        }
        CholWG0& z = *reinterpret_cast<CholWG0*>(tiles);
        uint32_t* bar12 = reinterpret_cast<uint32_t*>(misc + 4);    // waves 1, 2, 5, 6 barrier counter (zeroed above)
        uint32_t* p2done = reinterpret_cast<uint32_t*>(misc + 5);   // L(j+2, j) of step j formed: j + 1 (zeroed above)
        uint32_t* c2cnt = reinterpret_cast<uint32_t*>(misc + 6);    // halves of L(j+2, j-1) in C2: 2 j after step j
        uint32_t n12 = 0;
        // wave 3: publish L(j, j), Li_j, L(j+1, j), L(j+2, j) of step j (parity q = j & 1)
        // What the owners need for column block j -- Li_j (into its place in Li), the panel L(j+1, j) (into its
        // place in L) and T(j+2, j) through block j-1 (into the slot (j+2, j) of A, which nothing reads any more:
        // row j+2 was fetched at step j; row 2 is still the Gram's there at step 0) -- is stored by the wave that
        // finishes it during step j (the factor's wavefront: Li_j; the look-ahead's: L(j+1, j); waves 1 and 5:
        // T(j+2, j))
        // and completed before the
        // step's last barrier. Wave 3, at the start of step j+1: release them, then the outputs of step j (L(j, j),
        // L(j+2, j) and the packed forms), which only later kernels read.
        auto publish = [&](int j) {
            const int q = j & 1;
            const size_t o = (size_t)CB * j;
            if (lane == 0) {
                publish_flag(flagL + j * nb + j, ep);
                // the release covers column j-1's operands (stored in step j); column nb-2 is credited in the last
                // step, column nb-1 by wave 0
                if (j >= 1 && j < nb - 1) credit(colcnt, j - 1);
            }
            store_tile_lower(L + o * r + o, r, z.dl[q], false, lane, 64);
            store_tile_op(Lp + (size_t)op_pair(j, j) * CB * CB, z.li[q], lane, 64);
            if (j + 1 < nb) store_tile_op(Lp + (size_t)op_pair(j + 1, j) * CB * CB, z.P1[q], lane, 64);
            if (j + 2 < nb) {
                wait_lds(p2done, (uint32_t)j + 1, err, dead, lim);   // L(j+2, j), formed by the look-ahead
                store_tile(L + (o + 2 * CB) * r + o, r, z.P2[q], lane, 64);
                store_tile_op(Lp + (size_t)op_pair(j + 2, j) * CB * CB, z.P2[q], lane, 64);
            }
        };
        // Waves 0 and 7 take turns: at step j one factors T(j, j) (wave 0 at even j), the other forms tile row j+1's
        // look-ahead beside it and so ends the step holding T(j+1, j+1) through block j -- the next step's tile, in
        // the registers of the wavefront that factors it.
        float* fq = misc + 64;                                      // per pair: q_c, q_{c+1}, L(c+1, c)
        uint32_t* fcnt = reinterpret_cast<uint32_t*>(misc + 7);     // the factor's pairs done: 16 j + p + 1
        f32x16 C;                                                   // T(j, j) (factor) or T(j+1, j+1) (look-ahead)
        if (w == 0) load_sym(C, z.D[0]);
        for (int j = 0; j < nb; ++j) {
            const int p = j & 1, pp = p ^ 1;
            const int wf = p ? 7 : 0, wr = 7 - wf;                  // this step's factor and look-ahead wavefronts
            const uint32_t fbase = (uint32_t)(CB / 2) * j;
            if (STAMP && tid == 0) stamps[1 + 4 * j] = stamp_clock();
            if (w == wf) {
                factor_pairs(C, pq, fq, fcnt, fbase, tau, z.dl[p], z.li[p], Li + (size_t)CB * j * CB);
                if (STAMP && lane == 0) stamps[4 + 4 * j] = stamp_clock();
                if (colcnt != nullptr && j == nb - 1) {
                    // the last column of the factor is Li_{nb-1} alone: packed, released and credited at once
                    store_tile_op(Lp + (size_t)op_pair(j, j) * CB * CB, z.li[p], lane, 64);
                    release();
                    if (lane == 0) credit(colcnt, j);
                }
                __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this step's Li_j stored
            } else if (w == wr && j + 1 < nb) {
                f32x16 T2;
                if (j == 0) {
                    load_sym(C, z.D[1]);
                    load_tr(T2, z.X1);
                } else {
                    // L(j+1, j-1) = T(j+1, j-1) Li_{j-1}^T (row j+1 as fetched at step j-1), for waves 2 and 3; then
                    // block j-1 on T(j+1, j+1) and T(j+1, j)
                    panel32_wave(z.P2[pp], z.R2[pp][1], z.li[pp]);
                    if (lane == 0)
                        __hip_atomic_store(p2done, (uint32_t)j, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                    row_setup(C, T2, z.R2[pp][3], z.R2[pp][2], z.P2[pp], z.P1[pp]);
                }
                row_pairs(C, T2, fq, fcnt, fbase, z.dl[p], z.P1[p], L + (size_t)CB * (j + 1) * r + CB * j, r, err,
                          dead, lim);
                if (STAMP && lane == 0) stamps[3 + 4 * j] = stamp_clock();
                __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this step's L(j+1, j) stored
            } else if (w == 3) {
                // wave 3 publishes the previous step
                if (j >= 1) publish(j - 1);
                if (colcnt != nullptr && j == nb - 1 && nb >= 2) {   // column nb-2's operands, stored just now
                    release();
                    if (lane == 0) credit(colcnt, nb - 2);
                }
                if (STAMP && lane == 0) stamps[2 + 5 * nb + j] = stamp_clock();
            } else if ((w == 1 || w == 2 || w == 5 || w == 6) && j + 2 < nb) {
                // waves 1, 2, 5, 6: tile row j+2 through block j-1 (rows 2 and 3 straight from the Gram), into R2[p].
                // The four fetch row j+2 (from step 2 on each its own parts, without a barrier); then L(j+2, j-1)
                // (waves 1 and 5, a row half each) and the block j-2 update of T(j+2, j+1) that its owner left
                // (waves 2 and 6); then block j-1 on T(j+2, j) (waves 1 and 5), T(j+2, j+1) (waves 2 and 6, once
                // both halves of L(j+2, j-1) are there) and the lower quadrants of T(j+2, j+2) (waves 1, 5 and 2).
                Tile* R2 = z.R2[p];
                const int hf = w >> 2;                                   // row half (waves 5 and 6)
                const bool side2 = (w & 3) == 2;                         // waves 2 and 6
                const int i2 = j + 2, wl = ((w & 3) - 1 + 2 * hf) * 64 + lane;
                const float* rowp = A + (size_t)CB * i2 * r;
                if (j <= 1) {
                    const int t0 = (j == 0) ? 1 : 0;     // row 2: T(2, 0..2) into R2[1..3]; row 3: T(3, 0..3)
                    load_tiles<4, 256>(&R2[t0], 4 - t0, r, 1u << (3 - t0), shift, wl,
                                       [&](int q) { return rowp + CB * (j - 1 + t0 + q); });
                } else {
                    if (lane == 0) wait_flag(flagT + i2, ep, err, dead, lim);
                    if (STAMP && w == 1 && lane == 0) stamps[2 + 6 * nb + j] = stamp_clock();
                    __builtin_amdgcn_wave_barrier();
                    // each wavefront fetches the parts of row j+2 that it alone reads and updates below: waves 1 and
                    // 5 their halves of T(j+2, j-1) and T(j+2, j) and quadrant (hf, hf) of T(j+2, j+2); waves 2 and 6
                    // their halves of T(j+2, j+1) and of H = L(j+2, j-2), wave 2 quadrant (1, 0) of T(j+2, j+2)
                    const float* hp = L + (size_t)CB * i2 * r + (size_t)CB * (j - 2);
                    const int t0 = side2 ? 2 : 0, t1 = side2 ? 4 : 1;
                    const float* s0 = rowp + CB * (j - 1 + t0);
                    const float* s1 = side2 ? hp : rowp + CB * (j - 1 + t1);
                    const float* s3 = rowp + CB * (j + 2);
                    const bool quad = !side2 || hf == 0;
                    const int qa = side2 ? 1 : hf, qb = side2 ? 0 : hf;
                    float4 v[5];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int e = lane + 64 * u, row = 16 * hf + (e >> 3), c4 = e & 7;
                        v[u] = *reinterpret_cast<const float4*>(s0 + (size_t)row * r + 4 * c4);
                        v[2 + u] = *reinterpret_cast<const float4*>(s1 + (size_t)row * r + 4 * c4);
                    }
                    const int qrow = 16 * qa + (lane >> 2), qc4 = 4 * qb + (lane & 3);
                    if (quad) v[4] = *reinterpret_cast<const float4*>(s3 + (size_t)qrow * r + 4 * qc4);
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int e = lane + 64 * u, row = 16 * hf + (e >> 3), c4 = e & 7;
                        float* d0 = &R2[t0][row][4 * c4];
                        float* d1 = &R2[t1][row][4 * c4];
                        d0[0] = v[u].x; d0[1] = v[u].y; d0[2] = v[u].z; d0[3] = v[u].w;
                        d1[0] = v[2 + u].x; d1[1] = v[2 + u].y; d1[2] = v[2 + u].z; d1[3] = v[2 + u].w;
                    }
                    if (quad) {
                        float* d3 = &R2[3][qrow][4 * qc4];
                        d3[0] = v[4].x; d3[1] = v[4].y; d3[2] = v[4].z; d3[3] = v[4].w;
                    }
                    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wavefront's parts are in LDS
                    __builtin_amdgcn_wave_barrier();
                }
                if (j <= 1) wave_group_barrier(bar12, 4 * ++n12, err, dead, lim);
                if (STAMP && w == 1 && lane == 0) stamps[2 + 7 * nb + j] = stamp_clock();
                if (j >= 1) {
                    if (!side2) {
                        if (hf) panel32_wave<0xC>(z.C2[p], R2[0], z.li[pp]);          // L(j+2, j-1)
                        else panel32_wave<0x3>(z.C2[p], R2[0], z.li[pp]);
                        // this half of L(j+2, j-1) is in LDS for waves 2 and 6 (two per step from step 1)
                        if (lane == 0) __hip_atomic_fetch_add(c2cnt, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                        // its half for the output and the later kernels (the owners form their own copy)
                        const size_t o = (size_t)CB * (j - 1);
                        store_tile_half(L + (o + 3 * CB) * r + o, r, z.C2[p], hf, lane);
                        store_tile_op_half(Lp + (size_t)op_pair(j + 2, j - 1) * CB * CB, z.C2[p], hf, lane);
                    } else if (j >= 2) {                                               // T(j+2, j+1), block j-2
                        if (hf) update32_wave_q<0xC>(R2[2], R2[2], R2[4], z.C2[pp]);
                        else update32_wave_q<0x3>(R2[2], R2[2], R2[4], z.C2[pp]);
                    }
                    if (j <= 1) wave_group_barrier(bar12, 4 * ++n12, err, dead, lim);
                    if (STAMP && w == 1 && lane == 0) stamps[2 + 8 * nb + j] = stamp_clock();
                    if (!side2) {
                        // T(j+2, j), block j-1 (for the owners, in the slot of A that nothing reads any more), then
                        // quadrant (0, 0) or (1, 1) of T(j+2, j+2)
                        if (hf) {
                            update32_wave_q<0xC>(R2[1], R2[1], z.C2[p], z.P1[pp]);
                            store_tile_half(A + (size_t)CB * (j + 2) * r + CB * j, r, R2[1], 1, lane);
                            update32_wave_q<0x8>(R2[3], R2[3], z.C2[p], z.C2[p]);
                        } else {
                            update32_wave_q<0x3>(R2[1], R2[1], z.C2[p], z.P1[pp]);
                            store_tile_half(A + (size_t)CB * (j + 2) * r + CB * j, r, R2[1], 0, lane);
                            update32_wave_q<0x1>(R2[3], R2[3], z.C2[p], z.C2[p]);
                        }
                    } else {
                        if (j >= 2) wait_lds(c2cnt, 2u * (uint32_t)j, err, dead, lim);  // L(j+2, j-1), both halves
                        wait_lds(p2done, (uint32_t)j, err, dead, lim);                 // L(j+1, j-1) formed
                        if (hf) {
                            update32_wave_q<0xC>(R2[2], R2[2], z.C2[p], z.P2[pp]);     // T(j+2, j+1)
                            if (STAMP && lane == 0) stamps[2 + 9 * nb + j] = stamp_clock();
                        } else {
                            update32_wave_q<0x3>(R2[2], R2[2], z.C2[p], z.P2[pp]);
                            update32_wave_q<0x4>(R2[3], R2[3], z.C2[p], z.C2[p]);      // T(j+2, j+2), (1, 0)
                        }
                    }
                }
                if (STAMP && w == 1 && lane == 0) stamps[2 + 4 * nb + j] = stamp_clock();
            }
            __syncthreads();
            // start the L2 write-back of this step's stores now; the publication at the next step's start then
            // finds the lines clean
            if (w == 4) asm volatile("buffer_wbl2 sc1" ::: "memory");
            if (STAMP && tid == 0) stamps[2 + 4 * j] = stamp_clock();
        }
        if (w == 3) publish(nb - 1);
        if (STAMP && tid == 0) stamps[1 + 4 * nb] = stamp_clock();
    } else {
        // Owner part: tile row i, tiles T(i, s..e-1) in LDS. rt[k - s] = T(i, k); pn[k - s] = L(k, j) of the current
        // column block for the part's columns k < i; li = Li_j; pin = L(i, j) when another part of the row holds
        // T(i, j). Each part runs blocks j until its tiles are done: the last part (which holds T(i, i)) to block
        // i-4, after which it hands T(i, i-3..i) to workgroup 0; an earlier part to block e-1, its last panel.
        // Every panel a block needs is formed here from its tile through block j-1 -- L(k, j) = T(k, j) Li_j^T --
        // and those tiles are published a block ahead: the part holding T(i, j+1) stores it (in its slot of A) and
        // raises flag (i, j+1) as soon as block j has updated it. So a block waits on one round of flags: workgroup
        // 0's block j (Li_j, the finished L(j+1, j), T(j+2, j)), the hand-over of row j+3 (T(j+3, j)) and the tiles
        // T(k, j) of rows k >= j+4 and, when another part holds it, T(i, j), all published during block j-1.
        const int i = oi, s = os, e = oe;
        const bool last = e == i + 1;
        const int jl = last ? i - 4 : e - 1;
        const int pw = owner_lds_tiles(nb, ow) / 2 - 1;
        Tile* rt = tiles;
        Tile* pn = tiles + pw;
        Tile& li = tiles[2 * pw];
        Tile& pin = tiles[2 * pw + 1];
        const int l16 = lane & 15, lk = lane >> 4, qd = w & 3, bi = qd >> 1, bj = qd & 1;
        const bool upq = (bi == 0 && bj == 1);
        for (int j = 0; j <= jl; ++j) {
            const bool q4 = w < 4;
            const bool mine = j >= s;                               // this part holds T(i, j): L(i, j) is its output
            const bool hand = last && j + 4 == i;                   // the block after which row i is handed over
            // the part's columns k < i updated by block j: [k0, ke) (at the hand-over block T(i, i-1) is left to
            // workgroup 0, so L(i-1, j) is not needed)
            const int k0 = j + 1 > s ? j + 1 : s;
            const int ke = last ? (hand ? i - 1 : i) : e;
            const int nk = ke > k0 ? ke - k0 : 0;
            const bool hst = STAMP && hand && tid == 0;             // the hand-over block's stamps
            const bool bst = STAMP && last && i == nb - 1 && tid == 0;  // the last row's stamps, every block
            uint64_t* bs = stamps + 2 + 16 * nb + 8 * j;
            if (w == 0) {
                const uint32_t* f = nullptr;
                if (lane == 0) {
                    f = flagL + j * nb + j;
                } else if (lane <= nk) {
                    const int k = k0 + lane - 1;
                    if (k == j + 3) f = k >= 4 ? flagT + k : nullptr;             // row 3 never had an owner
                    else if (k >= j + 4 && j >= 1) f = flagL + k * nb + j;         // (block 0: the Gram's tiles)
                } else if (lane == nk + 1 && !mine && j >= 1) {
                    f = flagL + i * nb + j;
                }
                wait_flags_wave(f, ep, err, dead, lim);
            }
            __syncthreads();
            if (hst) stamps[2 + 10 * nb + 6 * i] = stamp_clock();
            if (bst) bs[0] = stamp_clock();
            // one batch: Li_j; per column k, the finished L(j+1, j) or T(k, j) through block j-1; T(i, j) into pin
            if (q4)
                load_tiles_to<OWNER_WMAX + 2, 256>(1 + nk + (mine ? 0 : 1), tid,
                                                [&](int q) -> Tile& { return q == 0 ? li : q <= nk ? pn[k0 + q - 1 - s] : pin; },
                                                [&](int q) {
                                                    if (q == 0) return (const float*)(Li + (size_t)CB * j * CB);
                                                    const int k = q <= nk ? k0 + q - 1 : i;
                                                    return (const float*)((k == j + 1 ? L : A) + (size_t)CB * k * r +
                                                                          (size_t)CB * j);
                                                },
                                                [&](int q) { return q == 0 ? CB : r; });   // Li_j's rows are 32 apart
            __syncthreads();
            if (hst) stamps[3 + 10 * nb + 6 * i] = stamp_clock();
            if (bst) bs[1] = stamp_clock();
            // the panels: L(i, j) (in place in rt[j - s] or pin) and L(k, j) for the columns k >= j+2
            Tile& lij = mine ? rt[j - s] : pin;
            const int kp = k0 > j + 2 ? k0 : j + 2;
            const int np = 1 + (ke > kp ? ke - kp : 0);
            panels_inplace(np, [&](int q) -> Tile& { return q == 0 ? lij : pn[kp + q - 1 - s]; }, li);
            if (hst) stamps[4 + 10 * nb + 6 * i] = stamp_clock();
            if (bst) bs[2] = stamp_clock();
            if (mine) {
                // L(i, j): the output, and its packed form for the solve (released below, with the column credit)
                if (q4) store_tile(L + (size_t)CB * i * r + (size_t)CB * j, r, lij);
                else store_tile_op(Lp + (size_t)op_pair(i, j) * CB * CB, lij, tid - 256, 256);
            } else if (hand && q4) {
                // workgroup 0 reads L(i, i-4) with the handed-over row: this part's own copy (the same bits as the
                // holder's), stored before the hand-over
                store_tile(L + (size_t)CB * i * r + (size_t)CB * j, r, lij);
            }
            // Row i's update by block j, every tile's quadrant chain in one phase (the tiles are independent): waves
            // w and w + 4 take quadrant (bi, bj) = (w & 3) of alternate tiles of a sequence (without the upper
            // quadrant of T(i, i)); the panel's A operands stay in registers, and the next tile's B operands and
            // accumulator are read while this tile's chain runs. T(i, j+1), which the next block's consumers wait
            // for, comes first.
            auto update_tiles = [&](int n, auto kof) {
                float an[8];
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) an[kk] = -lij[16 * bi + l16][4 * kk + lk];
                auto fetch = [&](int k, float (&bv)[8], f32x4& acc) {
                    const Tile& Pk = (k == i) ? lij : pn[k - s];
#pragma unroll
                    for (int kk = 0; kk < 8; ++kk) bv[kk] = Pk[16 * bj + l16][4 * kk + lk];
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[v] = rt[k - s][16 * bi + 4 * lk + v][16 * bj + l16];
                };
                // two operand sets in turn: tile t's chain runs while the operands of this wave's next tile are in
                // flight; the prefetch is unconditional (past the last tile it reads tile t again, unused), so the
                // wait before a chain only ever covers the previous prefetch
                auto chain = [&](int k, const float (&bv)[8], f32x4 acc) {
#pragma unroll
                    for (int kk = 0; kk < 8; ++kk) acc = mfma(an[kk], bv[kk], acc);
#pragma unroll
                    for (int v = 0; v < 4; ++v) rt[k - s][16 * bi + 4 * lk + v][16 * bj + l16] = acc[v];
                };
                // In-order issue: the next tile's reads go between the chain's first MFMAs (two after each), where
                // they issue while the previous MFMA runs and complete before the chain ends.
                auto interleave = [&]() {
#pragma unroll
                    for (int g = 0; g < 3; ++g) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // LDS reads
                    }
                    __builtin_amdgcn_sched_group_barrier(0x008, 5, 0);
                };
                int t = w >> 2;                 // this wave's tiles: t, t + 2, ...
                float b0[8], b1[8];
                f32x4 c0, c1;
                if (t < n) fetch(kof(t), b0, c0);
                while (t < n) {
                    int tn = t + 2;
                    fetch(kof(tn < n ? tn : t), b1, c1);
                    chain(kof(t), b0, c0);
                    interleave();
                    t = tn;
                    if (t >= n) break;
                    tn = t + 2;
                    fetch(kof(tn < n ? tn : t), b0, c0);
                    chain(kof(t), b1, c1);
                    interleave();
                    t = tn;
                }
            };
            // T(i, k0..ke-1), then T(i, i)
            update_tiles(nk + (last && !upq ? 1 : 0), [&](int t) { return k0 + t < ke ? k0 + t : i; });
            // this block's stores complete before the barrier, so that wave 7's release covers them (at the
            // hand-over the hand-over's own wait does)
            if (!hand) __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
            __syncthreads();
            if (hst) stamps[6 + 10 * nb + 6 * i] = stamp_clock();
            if (bst) bs[3] = stamp_clock();
            if (hand) {
                // hand T(i, i-3..i) to workgroup 0
                for (int t = 0; t < 4; ++t)
                    store_tile(A + (size_t)CB * i * r + (size_t)CB * (i - 3 + t), r, rt[i - 3 + t - s]);
                __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();
                if (hst) stamps[7 + 10 * nb + 6 * i] = stamp_clock();
                if (tid == 0) {
                    publish_flag(flagT + i, ep);
                    if (mine) credit(colcnt, j);   // L(i, i-4)'s packed form
                }
                if (hst) stamps[5 + 10 * nb + 6 * i] = stamp_clock();
            } else if (w == 7) {
                // T(i, j+1) through block j for the next block's consumers, and the column credit for L(i, j);
                // the other waves go on to the next block's wait meanwhile
                const bool pub = j + 1 >= s && j + 1 < e && j + 1 <= i - 4;
                if (pub) store_tile(A + (size_t)CB * i * r + (size_t)CB * (j + 1), r, rt[j + 1 - s], lane, 64);
                if (pub || mine) {
                    release();
                    if (lane == 0) {
                        if (pub) set_flag(flagL + i * nb + j + 1, ep);
                        if (mine) credit(colcnt, j);
                    }
                }
                if (STAMP && last && i == nb - 1 && lane == 0) bs[4] = stamp_clock();
            }
        }
    }
    __syncthreads();
    if (tid == 0) cnt[b] = ep;
}

// tau_ptr (nnp == 0 only; may be null): the absolute pivot floor read from device memory instead of tau_rel (chol32
// with tau as a device tensor, kchol.py:24-28: no host synchronisation)
template <bool STAMP>
__global__ __launch_bounds__(512) void k_chol(float* A, int r, const double* __restrict__ npart, int nnp, float alpha,
                                              float tau_rel, float* L, float* Li, float* Lp, uint32_t* bar,
                                              uint32_t* flags, float* scal, uint64_t* stamps, uint32_t lim, int ow,
                                              const float* tau_ptr) {
    chol_body<STAMP>(blockIdx.x, blockIdx.z, A, r, npart, nnp, alpha, tau_rel, L, Li, Lp, bar, flags, scal, stamps,
                     lim, nullptr, ow, tau_ptr);
}

// ---------------------------------------------------------------------------------------------------------------
// Triangular solve Y = A L^-T (tri.py:378-412). A workgroup of eight wavefronts takes RB blocks of 16 rows; wave w
// owns the 32-column blocks j = w, w+8, ... of all of them and keeps their accumulators (acc_j starts at a_j; pass 1:
// fmaf(eps, z, s * x)). For k = 0..nbc-1 the owner of block k forms Y_k = acc_k Li_k^T (chain over
// m < 16 (c/16 + 1)), publishes it in LDS behind a flag, and every wave applies it to its later blocks:
// acc_j -= Y_k L_jk^T (chain over the 32 columns of block k), so each element's chain runs over m = 0..32j-1 in
// order. Waves synchronise only through those per-block flags (bounded waits); each wave prefetches the L and Li
// operands of step k+1 into registers while it works on step k. The operands come packed (store_tile_op), as the
// Cholesky writes them: each lane reads its 16 values of a block with four 16-byte loads.
// ---------------------------------------------------------------------------------------------------------------
constexpr uint32_t FLAG_SPIN_LIMIT = 1u << 22;

// A solve running in the Cholesky's launch writes Y with agent-scope (write-through) stores, so that the lines are not
// left dirty in the L2 of an XCD whose Cholesky workgroups release there (a release writes every dirty line back)
__device__ __forceinline__ void store_wt(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int Q>
struct TrsmOps {
    float l[Q][2][8];    // L_jk B operands: [owned block][column half][kk]
};

// the 16 B operands of one packed factor block for this lane: o[cb][kk] (4 x 16-byte loads)
__device__ __forceinline__ void fetch_op(float (&o)[2][8], const float* __restrict__ Lp, int a, int b, int lane) {
    const float4* src = reinterpret_cast<const float4*>(Lp + (size_t)op_pair(a, b) * CB * CB + 16 * lane);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const float4 v = src[h];
        o[h >> 1][4 * (h & 1) + 0] = v.x;
        o[h >> 1][4 * (h & 1) + 1] = v.y;
        o[h >> 1][4 * (h & 1) + 2] = v.z;
        o[h >> 1][4 * (h & 1) + 3] = v.w;
    }
}

// Li_k B operands (block-lower: only kk < 4 (cb + 1) are used) for the owner of block k
__device__ __forceinline__ void trsm_fetch_li(float (&li)[2][8], const float* __restrict__ Lp, int nbc, int k,
                                              int lane) {
    if (k >= nbc) return;
    fetch_op(li, Lp, k, k, lane);
}

constexpr int TRSM_NW = 8;   // wavefronts per k_trsm workgroup; wave w owns the column blocks w + TRSM_NW q
// column blocks per wavefront for nb 32-column blocks: 1 (r <= 256), 2 (r <= 512) or 4 (r <= 1024)
constexpr int trsm_q_for(int nb) { return nb <= TRSM_NW ? 1 : nb <= 2 * TRSM_NW ? 2 : 4; }

template <int Q>
__device__ __forceinline__ void trsm_fetch(TrsmOps<Q>& o, const float* __restrict__ Lp, int nbc, int k, int w,
                                           int lane) {
    if (k >= nbc) return;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int j = w + TRSM_NW * q;
        if (j > k && j < nbc) fetch_op(o.l[q], Lp, j, k, lane);
    }
}

// WAIT (the solve in the Cholesky's launch): the operands of column block k are read only once its counter in
// colcnt has all its credits (see chol_body); wave 0 polls the counters in order, acquires, and raises an LDS word
// the other waves poll. Li_k is then fetched with column k's operands rather than eight steps ahead. A poll that
// gives up (after `lim` sleeps) records the error in err and proceeds, so the kernel always ends.
template <bool PASS1, int Q, int RB, bool WAIT>
__device__ __forceinline__ void trsm_body(const int rbi, const int z, const MatsIn& As, long lda, int K, int r,
                                          const uint32_t* __restrict__ amax_part, const float* __restrict__ Z,
                                          long ldz, float eps, const float* __restrict__ Lp, const MatsOut& Ys,
                                          long ldy, float* scal, const uint32_t* colcnt, uint32_t* err, uint32_t lim) {
    extern __shared__ float smem[];
    const float* __restrict__ A = As.p[z];
    float* __restrict__ Y = Ys.p[z];
    amax_part += (size_t)z * AMAX_BLOCKS;
    Lp += (size_t)z * (r / CB) * (r / CB + 1) / 2 * CB * CB;
    if (scal != nullptr) scal += (size_t)z * SCAL_STRIDE;
    const int ldsy = r + 4;
    float* sY = smem;                          // [16 RB][r + 4]: finished Y columns (MFMA A operands)
    float* sAcc = sY + 16 * RB * ldsy;         // [TRSM_NW][16][33]: per-wave transpose of the block being finished
    uint32_t* sFlag = reinterpret_cast<uint32_t*>(sAcc + TRSM_NW * 16 * 33);   // [nbc]
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, l16 = lane & 15, lk = lane >> 4;
    const int row0 = rbi * 16 * RB, nbc = r / CB;
    uint32_t* sReady = sFlag + nbc;            // WAIT: highest column block known complete, + 1
    if (WAIT) {
        colcnt += (size_t)z * CC_STRIDE * CH_MAXROW;
        err += (size_t)z * BAR_STRIDE;
    }
    float sc = 1.0f;
    if (PASS1) {
        sc = block_scale512(amax_part);
        if (rbi == 0 && tid == 0 && scal != nullptr) scal[0] = sc;
    }
    for (int k = tid; k < nbc; k += 64 * TRSM_NW) sFlag[k] = 0u;
    if (WAIT && tid == 0) *sReady = 0u;
    f32x4 acc[RB][Q][2];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int j = w + TRSM_NW * q;
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = row0 + 16 * rb + 4 * lk + v, col = CB * j + 16 * cb + l16;
                    float x = 0.0f;
                    if (j < nbc && row < K) {
                        x = A[(size_t)row * lda + col];
                        if (PASS1) x = __builtin_fmaf(eps, Z[(size_t)row * ldz + col], sc * x);
                    }
                    acc[rb][q][cb][v] = x;
                }
        }
    __syncthreads();   // flags cleared
    // WAIT: column blocks < known are complete as far as this wave knows
    int known = 0;
    bool dead = false;
    auto need_col = [&](int k) {
        if (!WAIT || k >= nbc || k < known) return;
        if (w == 0) {
            if (lane == 0) {
                for (int c = known; c <= k; ++c) {
                    const uint32_t want = 1u + (uint32_t)(nbc - 4 - c > 0 ? nbc - 4 - c : 0);
                    uint32_t n = 0;
                    while (!dead && __hip_atomic_load(colcnt + (size_t)c * CC_STRIDE, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT) < want) {
                        if (++n > lim) {
                            __hip_atomic_store(err + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            dead = true;
                            break;
                        }
                        __builtin_amdgcn_s_sleep(12);
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (lane == 0) __hip_atomic_store(sReady, (uint32_t)(k + 1), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        } else {
            uint32_t n = 0;
            while (__hip_atomic_load(sReady, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < (uint32_t)(k + 1)) {
                if (++n > FLAG_SPIN_LIMIT) break;
                __builtin_amdgcn_s_sleep(1);
            }
        }
        known = k + 1;
    };
    TrsmOps<Q> cur, nxt;
    float li[2][8];   // Li of this wave's next block to finish
    need_col(0);
    trsm_fetch<Q>(cur, Lp, nbc, 0, w, lane);
    if (WAIT) {
        if (w == 0) trsm_fetch_li(li, Lp, nbc, 0, lane);
    } else {
        trsm_fetch_li(li, Lp, nbc, w, lane);   // fetched TRSM_NW steps ahead
    }
    const bool full = row0 + 16 * RB <= K;   // every row of the workgroup exists: stores need no bounds check
    // finish block k (owner only): Y_k = acc_k Li_k^T into sY and Y, then raise its flag. The accumulator goes
    // through LDS into the MFMA A layout; both 16-column halves' chains run interleaved before any store.
    auto finish = [&](int k, int qk) {
        float* sa = sAcc + w * 16 * 33;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int v = 0; v < 4; ++v) sa[(4 * lk + v) * 33 + 16 * cb + l16] = acc[rb][qk][cb][v];
            __builtin_amdgcn_wave_barrier();
            float av[8];
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) av[kk] = sa[l16 * 33 + 4 * kk + lk];
            __builtin_amdgcn_sched_barrier(0);
            f32x4 y[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                if (kk < 4) y[0] = mfma(av[kk], li[0][kk], y[0]);
                y[1] = mfma(av[kk], li[1][kk], y[1]);
            }
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int rl = 16 * rb + 4 * lk + v, col = CB * k + 16 * cb + l16;
                    sY[rl * ldsy + col] = y[cb][v];
                    if (full || row0 + rl < K) {
                        if (WAIT) store_wt(&Y[(size_t)(row0 + rl) * ldy + col], y[cb][v]);
                        else Y[(size_t)(row0 + rl) * ldy + col] = y[cb][v];
                    }
                }
            __builtin_amdgcn_wave_barrier();
        }
        if (lane == 0) __hip_atomic_store(&sFlag[k], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (!WAIT) trsm_fetch_li(li, Lp, nbc, k + TRSM_NW, lane);
    };
    // acc_j -= Y_k L_jk^T for owned block q
    auto apply = [&](int k, int q) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            float av[8];   // the A operands read together, then both halves' chains interleaved
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) av[kk] = -sY[(16 * rb + l16) * ldsy + CB * k + 4 * kk + lk];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kk = 0; kk < 8; ++kk)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) acc[rb][q][cb] = mfma(av[kk], cur.l[q][cb][kk], acc[rb][q][cb]);
        }
    };
    if (w == 0) finish(0, 0);
#pragma unroll
    for (int qk = 0; qk < Q; ++qk) {
#pragma unroll
        for (int ow = 0; ow < TRSM_NW; ++ow) {
            const int k = TRSM_NW * qk + ow;
            if (k < nbc) {
                need_col(k + 1);
                trsm_fetch<Q>(nxt, Lp, nbc, k + 1, w, lane);
                if (WAIT && k + 1 < nbc && w == (k + 1) % TRSM_NW) trsm_fetch_li(li, Lp, nbc, k + 1, lane);
                if (w != ow) {
                    uint32_t n = 0;
                    while (__hip_atomic_load(&sFlag[k], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0u) {
                        if (++n > FLAG_SPIN_LIMIT) break;
                        __builtin_amdgcn_s_sleep(1);
                    }
                }
                // the owner of block k+1 brings it up to date and publishes it before its other updates
                const int kn = k + 1;
#pragma unroll
                for (int q = 0; q < Q; ++q) {
                    const int j = w + TRSM_NW * q;
                    if (j == kn && j < nbc) apply(k, q);
                }
#pragma unroll
                for (int q = 0; q < Q; ++q) {
                    const int j = w + TRSM_NW * q;
                    if (j == kn && j < nbc) finish(kn, q);
                }
#pragma unroll
                for (int q = 0; q < Q; ++q) {
                    const int j = w + TRSM_NW * q;
                    if (j > kn && j < nbc) apply(k, q);
                }
                cur = nxt;
            }
        }
    }
}

template <bool PASS1, int Q, int RB>
__global__ __launch_bounds__(64 * TRSM_NW) void k_trsm(const MatsIn As, long lda, int K, int r,
                                              const uint32_t* __restrict__ amax_part, const float* __restrict__ Z,
                                              long ldz, float eps, const float* __restrict__ Lp, const MatsOut Ys,
                                              long ldy, float* scal) {
    trsm_body<PASS1, Q, RB, false>(blockIdx.x, blockIdx.z, As, lda, K, r, amax_part, Z, ldz, eps, Lp, Ys, ldy, scal,
                                   nullptr, nullptr, 0);
}

// The solve for tall X in the Cholesky's launch: each wavefront owns one block of 16 rows and all r/32 = NBC column
// blocks (accumulators in registers) and runs right-looking through the column blocks as the factor's columns become
// complete: Y_k = acc_k Li_k^T, then acc_j -= Y_k L_jk^T for every j > k. Same arithmetic, element by element, as
// k_trsm (acc_j starts at a_j, or fmaf(eps, z, s x) on pass 1; its updates by k ascending, each one MFMA chain over
// the 32 columns of block k; the product with Li_k a chain over m < 16 (c/16 + 1)). No wavefront waits on another but
// for column readiness (wave 0 polls the counters, the others an LDS word), so after the factor's last column only
// one block product remains. Workgroup g of a matrix takes row blocks wpg g .. wpg g + wpg - 1 (wpg <= 8: the plan
// spreads the row blocks over every CU the Cholesky leaves free, one workgroup per CU, so that fewer wavefronts
// share a SIMD); waves past wpg or past K have no work.
template <bool PASS1, int NBC>
__device__ __forceinline__ void trsm_wave_body(const int g, const int z, const MatsIn& As, long lda, int K, int wpg,
                                               const uint32_t* __restrict__ amax_part, const float* __restrict__ Z,
                                               long ldz, float eps, const float* __restrict__ Lp, const MatsOut& Ys,
                                               long ldy, float* scal, const uint32_t* colcnt, uint32_t* err,
                                               uint32_t lim) {
    extern __shared__ float smem[];
    const float* __restrict__ A = As.p[z];
    float* __restrict__ Y = Ys.p[z];
    amax_part += (size_t)z * AMAX_BLOCKS;
    Lp += (size_t)z * NBC * (NBC + 1) / 2 * CB * CB;
    if (scal != nullptr) scal += (size_t)z * SCAL_STRIDE;
    colcnt += (size_t)z * CC_STRIDE * CH_MAXROW;
    err += (size_t)z * BAR_STRIDE;
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, l16 = lane & 15,
              lk = lane >> 4;
    float* sT = smem + w * 16 * 33;                                       // this wave's transpose tile
    uint32_t* sReady = reinterpret_cast<uint32_t*>(smem + TRSM_NW * 16 * 33);
    float sc = 1.0f;
    if (PASS1) {
        sc = block_scale512(amax_part);
        if (g == 0 && tid == 0 && scal != nullptr) scal[0] = sc;
    }
    if (tid == 0) *sReady = 0u;
    __syncthreads();
    const int row0 = (g * wpg + w) * 16;
    if (w != 0 && (w >= wpg || row0 >= K)) return;   // wave 0 (always in range) is the poller
    const bool live = w < wpg && row0 < K;
    // rows past K read row K-1 (in bounds) and are zeroed
    int rowc[4];
    bool rin[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int row = row0 + 4 * lk + v;
        rin[v] = row < K;
        rowc[v] = rin[v] ? row : K - 1;
    }
    f32x4 acc[NBC][2];
#pragma unroll
    for (int j = 0; j < NBC; ++j)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int col = CB * j + 16 * cb + l16;
                float x = A[(size_t)rowc[v] * lda + col];
                if (PASS1) x = __builtin_fmaf(eps, Z[(size_t)rowc[v] * ldz + col], sc * x);
                acc[j][cb][v] = rin[v] ? x : 0.0f;
            }
    bool dead = false;
#pragma unroll
    for (int k = 0; k < NBC; ++k) {
        // column block k of the factor complete (Li_k and L(j, k) for every j > k)
        if (w == 0) {
            if (lane == 0) {
                const uint32_t want = 1u + (uint32_t)(NBC - 4 - k > 0 ? NBC - 4 - k : 0);
                uint32_t n = 0;
                while (!dead && __hip_atomic_load(colcnt + (size_t)k * CC_STRIDE, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT) < want) {
                    if (++n > lim) {
                        __hip_atomic_store(err + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        dead = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(12);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (lane == 0) __hip_atomic_store(sReady, (uint32_t)(k + 1), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (!live) continue;
        } else {
            uint32_t n = 0;
            while (__hip_atomic_load(sReady, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < (uint32_t)(k + 1)) {
                if (++n > FLAG_SPIN_LIMIT) break;
                __builtin_amdgcn_s_sleep(1);
            }
        }
        // the column's operands: Li_k, then L(j, k) for j > k (each 16 floats per lane, packed)
        float li[2][8];
        fetch_op(li, Lp, k, k, lane);
        float lo[NBC][2][8];
#pragma unroll
        for (int j = k + 1; j < NBC; ++j) fetch_op(lo[j], Lp, j, k, lane);
        // Y_k = acc_k Li_k^T: the accumulator through LDS into the MFMA A layout
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int v = 0; v < 4; ++v) sT[(4 * lk + v) * 33 + 16 * cb + l16] = acc[k][cb][v];
        __builtin_amdgcn_wave_barrier();
        float av[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) av[kk] = sT[l16 * 33 + 4 * kk + lk];
        __builtin_amdgcn_sched_barrier(0);
        f32x4 y[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            if (kk < 4) y[0] = mfma(av[kk], li[0][kk], y[0]);
            y[1] = mfma(av[kk], li[1][kk], y[1]);
        }
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (rin[v]) store_wt(&Y[(size_t)(row0 + 4 * lk + v) * ldy + CB * k + 16 * cb + l16], y[cb][v]);
                sT[(4 * lk + v) * 33 + 16 * cb + l16] = y[cb][v];
            }
        if (k + 1 < NBC) {
            // Y_k as the A operand of the later blocks' updates
            __builtin_amdgcn_wave_barrier();
            float ya[8];
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) ya[kk] = -sT[l16 * 33 + 4 * kk + lk];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = k + 1; j < NBC; ++j)
#pragma unroll
                for (int kk = 0; kk < 8; ++kk)
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) acc[j][cb] = mfma(ya[kk], lo[j][cb][kk], acc[j][cb]);
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// One pass's Cholesky and its solve in one launch: workgroups [0, nz grid) run the Cholesky of matrix
// b / grid (workgroup b % grid), the rest the solve of matrix b' / nrb (row blocks of 16 RB rows, b' % nrb), the
// solve following the factor column by column through the counters (the Cholesky's workgroups come first, so they
// are dispatched first and never wait on a solve workgroup). Pointers address matrix 0 of the launch.
struct CholArgs {
    float* A; const double* npart; float* L; float* Li; float* Lp; uint32_t* bar; uint32_t* flags; float* scal;
    uint32_t* colcnt; float alpha, tau_rel; int r, nnp, nz, grid, ow; uint32_t lim;   // ow: owner part width
};
struct SolveArgs {
    MatsIn A; MatsOut Y; const uint32_t* amax_part; const float* Z; float* scal; long lda, ldz, ldy; float eps;
    int K, nrb, wpg;   // wpg: row blocks (wavefronts) per workgroup of the one-wavefront-per-row-block solve
};

// Q > 0: the solve of k_trsm (Q column blocks per wave, RB row blocks of 16 per workgroup); Q = 0: trsm_wave_body
// with NBC = RB column blocks (eight row blocks per workgroup).
template <bool PASS1, int Q, int RB>
__global__ __launch_bounds__(64 * TRSM_NW) void k_chol_solve(const CholArgs c, const SolveArgs t) {
    const int nchol = c.nz * c.grid;
    if ((int)blockIdx.x < nchol) {
        chol_body<false>(blockIdx.x % c.grid, blockIdx.x / c.grid, c.A, c.r, c.npart, c.nnp, c.alpha, c.tau_rel, c.L,
                         c.Li, c.Lp, c.bar, c.flags, c.scal, nullptr, c.lim, c.colcnt, c.ow);
        return;
    }
    const int b = blockIdx.x - nchol;
    if constexpr (Q == 0)
        trsm_wave_body<PASS1, RB>(b % t.nrb, b / t.nrb, t.A, t.lda, t.K, t.wpg, t.amax_part, t.Z, t.ldz, t.eps, c.Lp, t.Y,
                                  t.ldy, t.scal, c.colcnt, c.bar, c.lim);
    else
        trsm_body<PASS1, Q, RB, true>(b % t.nrb, b / t.nrb, t.A, t.lda, t.K, c.r, t.amax_part, t.Z, t.ldz, t.eps,
                                      c.Lp, t.Y, t.ldy, t.scal, c.colcnt, c.bar, c.lim);
}

// Triangular solve with a workgroup of two wavefronts per 16 rows (r = 32 NBC <= 256, tall X): wavefront h takes the
// 16-column half h of every column block, in order, left-looking: acc_j = A_j - sum_{k<j} Y_k L_jk^T (one MFMA chain
// per element, k and then m ascending, the order of the blocked solve), then Y_j = acc_j Li_j^T. The product's A
// operand spans the block's 32 columns, so the pair swaps its accumulator halves through LDS, and then Y_j, which
// both keep in registers as the later blocks' MFMA A operands (one workgroup barrier each). Two wavefronts per row
// tile halve each chain, and the resulting ~2 wavefronts per SIMD at the tall shapes overlap one's LDS traffic with
// the other's MFMAs. The packed L operands (each wavefront its half) stream from L2 three blocks ahead of use
// (scheduling barriers keep the loads where they are issued), and A one column block ahead. The arithmetic of every
// element is that of k_trsm.
template <bool PASS1, int NBC>
__global__ __launch_bounds__(128) void k_trsm_rows(const MatsIn As, long lda, int K,
                                                   const uint32_t* __restrict__ amax_part, const float* __restrict__ Z,
                                                   long ldz, float eps, const float* __restrict__ Lp, const MatsOut Ys,
                                                   long ldy, float* scal) {
    constexpr int NSTEP = NBC * (NBC + 1) / 2;   // operand blocks in use order: L(j, 0..j-1), then Li_j, per j
    constexpr int DIST = 3;                       // operand blocks in flight ahead of the one in use
    __shared__ float sT[2][16][33];               // the pair's exchange: [0] acc_j, [1] Y_j (16 rows x 32 columns)
    const int z = blockIdx.z;
    const float* __restrict__ A = As.p[z];
    float* __restrict__ Y = Ys.p[z];
    amax_part += (size_t)z * AMAX_BLOCKS;
    Lp += (size_t)z * NSTEP * CB * CB;
    const int tid = threadIdx.x, h = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, l16 = lane & 15,
              lk = lane >> 4;
    float sc = 1.0f;
    if (PASS1) {
        sc = block_scale128(amax_part);
        if (blockIdx.x == 0 && tid == 0 && scal != nullptr) scal[(size_t)z * SCAL_STRIDE] = sc;
    }
    const int row0 = blockIdx.x * 16;   // < K: the grid is ceil(K / 16)
    // rows past K read row K-1 (in bounds) and are zeroed, so every load is unconditional
    int rowc[4];
    bool rin[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int row = row0 + 4 * lk + v;
        rin[v] = row < K;
        rowc[v] = rin[v] ? row : K - 1;
    }
    // this wavefront's half of the packed operand blocks, in use order; block s is consumed at step s and fetched at
    // step s - DIST (packed layout: 16 floats per lane, the half h at 8 h)
    float ob[DIST + 1][8];
    auto fetch_step = [&](int sidx) {
        int j = 0;
        while ((j + 1) * (j + 2) / 2 <= sidx) ++j;
        const int k = sidx - j * (j + 1) / 2;
        const float4* src = reinterpret_cast<const float4*>(Lp + (size_t)op_pair(j, k) * CB * CB + 16 * lane + 8 * h);
        float(&o)[8] = ob[sidx % (DIST + 1)];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const float4 v = src[q];
            o[4 * q + 0] = v.x;
            o[4 * q + 1] = v.y;
            o[4 * q + 2] = v.z;
            o[4 * q + 3] = v.w;
        }
        __builtin_amdgcn_sched_barrier(0);   // keep the prefetch where it is issued (the scheduler would sink it)
    };
    // this wavefront's half of A_j (and Z_j on pass 1) in C layout, one block ahead
    float xa[2][4], za[2][4];
    auto fetch_x = [&](int j, int buf) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int col = CB * j + 16 * h + l16;
            xa[buf][v] = A[(size_t)rowc[v] * lda + col];
            if (PASS1) za[buf][v] = Z[(size_t)rowc[v] * ldz + col];
        }
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int q = 0; q < DIST; ++q)
        if (q < NSTEP) fetch_step(q);
    fetch_x(0, 0);
    float ya[NBC][8];                 // ya[k][kk] = Y[row0 + l16][32 k + 4 kk + lk], both halves
    int sidx = 0;
#pragma unroll
    for (int j = 0; j < NBC; ++j) {
        if (j + 1 < NBC) fetch_x(j + 1, (j + 1) & 1);
        f32x4 acc;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            float x = xa[j & 1][v];
            if (PASS1) x = __builtin_fmaf(eps, za[j & 1][v], sc * x);
            acc[v] = rin[v] ? x : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < j; ++k) {
            if (sidx + DIST < NSTEP) fetch_step(sidx + DIST);
            const float(&o)[8] = ob[sidx % (DIST + 1)];
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) acc = mfma(-ya[k][kk], o[kk], acc);
            ++sidx;
        }
        if (sidx + DIST < NSTEP) fetch_step(sidx + DIST);
        const float(&li)[8] = ob[sidx % (DIST + 1)];
        ++sidx;
        // Y_j = acc_j Li_j^T: the product's A operand is acc_j over the block's 32 columns, from both wavefronts
#pragma unroll
        for (int v = 0; v < 4; ++v) sT[0][4 * lk + v][16 * h + l16] = acc[v];
        __syncthreads();
        float ar[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) ar[kk] = sT[0][l16][4 * kk + lk];
        f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            if (kk < 4 * (h + 1)) y = mfma(ar[kk], li[kk], y);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            if (rin[v]) Y[(size_t)(row0 + 4 * lk + v) * ldy + CB * j + 16 * h + l16] = y[v];
            sT[1][4 * lk + v][16 * h + l16] = y[v];
        }
        __syncthreads();
        if (j + 1 < NBC) {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) ya[j][kk] = sT[1][l16][4 * kk + lk];
        }
    }
}

// The packed solve operands (store_tile_op's layout) from row-major L [r, r] and Li [r, 32], for the stage entry
// point; one thread per packed element.
__global__ __launch_bounds__(256) void k_pack_factors(const float* __restrict__ L, const float* __restrict__ Li, int r,
                                                      float* __restrict__ Lp) {
    const int nb = r / CB, npairs = nb * (nb + 1) / 2;
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= npairs * CB * CB) return;
    const int pr = e >> 10, lane = (e >> 4) & 63, cb = (e >> 3) & 1, kk = e & 7;
    int a = 0;
    while (op_pair(a + 1, 0) <= pr) ++a;
    const int b = pr - op_pair(a, 0);
    const int row = 16 * cb + (lane & 15), col = 4 * kk + (lane >> 4);
    Lp[e] = (a == b) ? Li[(size_t)(CB * a + row) * CB + col] : L[(size_t)(CB * a + row) * r + CB * b + col];
}

// ---------------------------------------------------------------------------------------------------------------
// Newton-Schulz apply (kcholqr.py:22, addmm(Y, Y, D)): Out = Y + fp32(Y D), the product an MFMA chain over
// m = 0..r-1 from 0 and added to Y once. 32x64 output tile per workgroup; wave w: rows 16(w >> 1), 2 column blocks.
// MS columns of Y (rows of D) per step through LDS (32 or 64).
// ---------------------------------------------------------------------------------------------------------------
// SUB (the block projection, kbig.py:88-89): Out = C - fp32(A B) with A [K, r] of another matrix and C its own input,
// B [r, ncols] (row stride ldd); the chain and the single rounding are the same. The Newton-Schulz step is
// A = C = Y, B = D.
// err (Newton-Schulz only; may be null): the matrix's wait-error word; when a bounded wait of the call's Cholesky
// gave up, the output is NaN, so the failure shows in Q without a host synchronisation. Out may alias Cin (the
// projection updates its block in place; each element is read before it is written, by the same thread).
template <bool SUB = false, int MS = 32>
__global__ __launch_bounds__(256) void k_nsapply(const MatsIn Ys, long ldy, int K, int r, const float* __restrict__ D,
                                                 const MatsOut Outs, long ldo, const float* Cx = nullptr,
                                                 long ldc = 0, long ldd = 0, const uint32_t* err = nullptr) {
    const float* __restrict__ Yin = Ys.p[blockIdx.z];
    float* Out = Outs.p[blockIdx.z];
    const long ldD = SUB ? ldd : r;
    D += (size_t)blockIdx.z * r * ldD;
    const bool failed = err != nullptr && err[(size_t)blockIdx.z * BAR_STRIDE + 2] != 0u;
    const float* Cin = SUB ? Cx : Yin;
    const long ldC = SUB ? ldc : ldy;
    // row strides 34 and 80: each half-wavefront's operand reads (A: rows l16, columns 4kk + lk; B: rows 4kk + lk,
    // columns l16) fall on 32 distinct banks
    __shared__ float sY[32][MS + 2];
    __shared__ float sD[MS][80];
    const int row0 = blockIdx.x * 32, col0 = blockIdx.y * 64;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, lk = lane >> 4;
    const int rb = w >> 1, cbase = (w & 1) * 2;
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    for (int m0 = 0; m0 < r; m0 += MS) {
#pragma unroll
        for (int q = 0; q < MS / 32; ++q) {
            const int idx = tid + 256 * q, row = idx / (MS / 4), c4 = idx % (MS / 4);
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row0 + row < K) v = *reinterpret_cast<const float4*>(Yin + (size_t)(row0 + row) * ldy + m0 + 4 * c4);
            sY[row][4 * c4 + 0] = v.x; sY[row][4 * c4 + 1] = v.y; sY[row][4 * c4 + 2] = v.z; sY[row][4 * c4 + 3] = v.w;
        }
#pragma unroll
        for (int q = 0; q < MS / 16; ++q) {
            const int idx = tid + 256 * q, row = idx >> 4, c4 = idx & 15;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            // columns past r (SUB: past ldd, B's columns; a multiple of 32) feed only outputs that are not written
            if (col0 + 4 * c4 < (SUB ? ldd : r))
                v = *reinterpret_cast<const float4*>(D + (size_t)(m0 + row) * ldD + col0 + 4 * c4);
            *reinterpret_cast<float4*>(&sD[row][4 * c4]) = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < MS / 4; ++kk) {
            const float a = sY[16 * rb + l16][4 * kk + lk];
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[c] = mfma(a, sD[4 * kk + lk][16 * (cbase + c) + l16], acc[c]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = row0 + 16 * rb + 4 * lk + v, col = col0 + 16 * (cbase + c) + l16;
            if (row < K && col < (SUB ? ldd : r)) {
                const float cv = Cin[(size_t)row * ldC + col];
                Out[(size_t)row * ldo + col] = failed ? __builtin_nanf("") : SUB ? cv - acc[c][v] : cv + acc[c][v];
            }
        }
}

// The Newton-Schulz step of k_nsapply (same tiles, chains and rounding, so the same bits) for grids of about one
// workgroup per CU, where no other workgroup hides a step's load latency: the MS-column steps go through two LDS
// buffers, and the global loads of step s + 3 are issued as step s ends, into one of two register sets, so each load
// has two steps of MFMA work to arrive in (one barrier per step).
template <int MS>
__global__ __launch_bounds__(256) void k_nsapply_pipe(const MatsIn Ys, long ldy, int K, int r,
                                                      const float* __restrict__ D, const MatsOut Outs, long ldo,
                                                      const uint32_t* err) {
    const float* __restrict__ Yin = Ys.p[blockIdx.z];
    float* __restrict__ Out = Outs.p[blockIdx.z];
    D += (size_t)blockIdx.z * r * r;
    const bool failed = err != nullptr && err[(size_t)blockIdx.z * BAR_STRIDE + 2] != 0u;
    __shared__ float sY[2][32][MS + 2];
    __shared__ float sD[2][MS][80];
    const int row0 = blockIdx.x * 32, col0 = blockIdx.y * 64;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, lk = lane >> 4;
    const int rb = w >> 1, cbase = (w & 1) * 2;
    constexpr int NY = MS / 32, ND = MS / 16;
    struct Regs { float4 y[NY], d[ND]; } R0, R1;
    const int ns = r / MS;
    auto gload = [&](int s, Regs& R) {
        const int m0 = s * MS;
#pragma unroll
        for (int q = 0; q < NY; ++q) {
            const int idx = tid + 256 * q, row = idx / (MS / 4), c4 = idx % (MS / 4);
            // unconditional loads from clamped (in-bounds) addresses: no branch between a step's loads, so the wait
            // before a register set's LDS store counts only the loads issued before it. Row i of Y feeds only output
            // row i, and column j of D only output column j, so rows past K and columns past r (r % 64 == 32) read
            // any in-bounds values: they reach only outputs that are not written.
            const int gr = row0 + row < K ? row0 + row : K - 1;
            R.y[q] = *reinterpret_cast<const float4*>(Yin + (size_t)gr * ldy + m0 + 4 * c4);
        }
#pragma unroll
        for (int q = 0; q < ND; ++q) {
            const int idx = tid + 256 * q, row = idx >> 4, c4 = idx & 15;
            const int gc = col0 + 4 * c4 < r ? col0 + 4 * c4 : 0;
            R.d[q] = *reinterpret_cast<const float4*>(D + (size_t)(m0 + row) * r + gc);
        }
    };
    auto lstore = [&](int buf, const Regs& R) {
#pragma unroll
        for (int q = 0; q < NY; ++q) {
            const int idx = tid + 256 * q, row = idx / (MS / 4), c4 = idx % (MS / 4);
            sY[buf][row][4 * c4 + 0] = R.y[q].x; sY[buf][row][4 * c4 + 1] = R.y[q].y;
            sY[buf][row][4 * c4 + 2] = R.y[q].z; sY[buf][row][4 * c4 + 3] = R.y[q].w;
        }
#pragma unroll
        for (int q = 0; q < ND; ++q) {
            const int idx = tid + 256 * q, row = idx >> 4, c4 = idx & 15;
            *reinterpret_cast<float4*>(&sD[buf][row][4 * c4]) = R.d[q];
        }
    };
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    // a step's LDS operands are read ahead of its MFMAs (two steps' worth in flight), so the LDS latency overlaps the
    // chains
    auto compute = [&](int buf) {
        float xa[MS / 4], xb[2][MS / 4];
#pragma unroll
        for (int kk = 0; kk < MS / 4; ++kk) {
            xa[kk] = sY[buf][16 * rb + l16][4 * kk + lk];
#pragma unroll
            for (int c = 0; c < 2; ++c) xb[c][kk] = sD[buf][4 * kk + lk][16 * (cbase + c) + l16];
        }
#pragma unroll
        for (int kk = 0; kk < MS / 4; ++kk)
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[c] = mfma(xa[kk], xb[c][kk], acc[c]);
        __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
        for (int g = 0; g < MS / 4 - 2; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    };
    // ns is even (checked at launch). Every load and LDS store is unconditional (steps past the last reload the last
    // step, whose copy in a buffer is never multiplied), so the loop body has no branch and each LDS store waits only
    // for its own register set
    const int last = ns - 1;
    gload(0, R0);
    gload(1, R1);
    lstore(0, R0);
    __syncthreads();
    // the residual's Y elements (this lane's outputs), fetched now so the epilogue does not wait for them
    float cv[2][4];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = row0 + 16 * rb + 4 * lk + v, col = col0 + 16 * (cbase + c) + l16;
            cv[c][v] = Yin[(size_t)(row < K ? row : K - 1) * ldy + (col < r ? col : 0)];
        }
    gload(min(2, last), R0);
    __builtin_amdgcn_sched_barrier(0);   // the loads go out here, not next to their LDS stores
    // steps s, s + 1: multiply from buffer 0 (1), move register set 1 (0) -- step s + 1 (s + 2) -- into the other
    // buffer, then refill that set with step s + 3 (s + 4)
    int s = 0;
    do {   // (a do-while: no guard before the loop, below which the set-1 loads above could be moved)
        compute(0);
        lstore(1, R1);
        __syncthreads();
        gload(min(s + 3, last), R1);
        __builtin_amdgcn_sched_barrier(0);
        compute(1);
        lstore(0, R0);
        __syncthreads();
        gload(min(s + 4, last), R0);
        __builtin_amdgcn_sched_barrier(0);
        s += 2;
    } while (s < ns);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = row0 + 16 * rb + 4 * lk + v, col = col0 + 16 * (cbase + c) + l16;
            if (row < K && col < r) Out[(size_t)row * ldo + col] = failed ? __builtin_nanf("") : cv[c][v] + acc[c][v];
        }
}

// The Newton-Schulz step for tall Y (same chains and rounding as k_nsapply, so the same bits), r % 64 == 0, r <= MAXR.
// Workgroup (slab, g) of nslab * G: its four wavefronts own the four 16-column tiles of 64-column slab `slab` and keep
// their MFMA B operands (the tile's r rows of D) in registers for the whole launch, so D is read once per workgroup
// instead of once per 32 rows; the workgroup walks 16-row blocks g, g + G, ... of Y through two LDS buffers, the
// next block's loads in flight during a block's chain. The four slabs of one row group sit on one XCD (workgroup id
// mod 8), so each Y row is fetched into one L2. LDS holds a block as [row][k mod 4][k / 4] (rows padded): the A
// operands of four consecutive MFMAs are one 16-byte read; the residual Y is read back from the same buffer.
// The two buffers are dynamic LDS: nsr_lds_bytes (35 KB for MAXR = 256, 67 KB for 512).
constexpr int NSR_PADK = 4;
template <int MAXR>
constexpr int nsr_row_stride() { return 4 * (MAXR / 4 + NSR_PADK) + 4; }
template <int MAXR>
constexpr size_t nsr_lds_bytes() { return (size_t)2 * 16 * nsr_row_stride<MAXR>() * sizeof(float); }
template <int MAXR>
__global__ __launch_bounds__(256, 2) void k_nsapply_res(const MatsIn Ys, long ldy, int K, int r,
                                                        const float* __restrict__ D, const MatsOut Outs, long ldo,
                                                        const uint32_t* err, int G) {
    constexpr int KS = MAXR / 4 + NSR_PADK, RS = nsr_row_stride<MAXR>();
    extern __shared__ __align__(16) float nsr_lds[];
    auto sY = [&](int buf) { return nsr_lds + buf * 16 * RS; };   // buffer buf
    const float* __restrict__ Yin = Ys.p[blockIdx.z];
    float* __restrict__ Out = Outs.p[blockIdx.z];
    D += (size_t)blockIdx.z * r * r;
    const bool failed = err != nullptr && err[(size_t)blockIdx.z * BAR_STRIDE + 2] != 0u;
    const int nslab = r / 64, id = blockIdx.x, rest = id >> 3;
    const int slab = rest % nslab, g = (id & 7) + 8 * (rest / nslab);
    const int nblk = (K + 15) / 16;
    if (g >= nblk) return;   // (the launch keeps G <= nblk; whole workgroup, before any barrier)
    const int nb = (nblk - g + G - 1) / G;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, lk = lane >> 4;
    const int c0 = slab * 64 + 16 * w, r4 = r / 4;
    // B operands: bD[kk] = D[4 kk + lk][c0 + l16] (kk >= r / 4 loads a valid row and is never multiplied)
    float bD[MAXR / 4];
#pragma unroll
    for (int kk = 0; kk < MAXR / 4; ++kk) bD[kk] = D[(size_t)(4 * (kk < r4 ? kk : r4 - 1) + lk) * r + c0 + l16];
    // Y block loads: float4 q of this thread is row qrow[q] = (tid + 256 q) / r4, columns 4 c4 .. 4 c4 + 3 with c4
    // the remainder (divided once, here)
    constexpr int NQ = MAXR / 64;
    float4 R[NQ];
    int qrow[NQ], qc4[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int idx = tid + 256 * q;
        qrow[q] = idx / r4;
        qc4[q] = idx - qrow[q] * r4;
    }
    auto gload = [&](int i) {
        const int row0 = (g + i * G) * 16;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            // rows past K (and past the block, q >= r / 64, never stored) read row K - 1: row i of Y feeds only
            // output row i, which is not written
            const int gr = row0 + qrow[q] < K ? row0 + qrow[q] : K - 1;
            R[q] = *reinterpret_cast<const float4*>(Yin + (size_t)gr * ldy + 4 * qc4[q]);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            if (q < r / 64) {
                float* d = &sY(buf)[qrow[q] * RS + qc4[q]];
                d[0] = R[q].x; d[KS] = R[q].y; d[2 * KS] = R[q].z; d[3 * KS] = R[q].w;
            }
        }
    };
    gload(0);
    lstore(0);
    __syncthreads();
    if (nb > 1) gload(1);
    for (int i = 0; i < nb; ++i) {
        const int buf = i & 1;
        const float* sb = &sY(buf)[l16 * RS + lk * KS];
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k0 = 0; k0 < MAXR / 4; k0 += 16) {
            if (k0 >= r4) break;
            float4 a[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const float4*>(sb + k0 + 4 * j);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc = mfma(a[j].x, bD[k0 + 4 * j + 0], acc);
                acc = mfma(a[j].y, bD[k0 + 4 * j + 1], acc);
                acc = mfma(a[j].z, bD[k0 + 4 * j + 2], acc);
                acc = mfma(a[j].w, bD[k0 + 4 * j + 3], acc);
            }
        }
        if (i + 1 < nb) lstore(buf ^ 1);   // its last readers finished before the previous barrier
        const int row0 = (g + i * G) * 16, col = c0 + l16;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = row0 + 4 * lk + v;
            const float cv = sY(buf)[(4 * lk + v) * RS + (col & 3) * KS + (col >> 2)];
            if (row < K) Out[(size_t)row * ldo + col] = failed ? __builtin_nanf("") : cv + acc[v];
        }
        __syncthreads();
        if (i + 2 < nb) gload(i + 2);
    }
}

// k_amax's block size: 1024 threads for X of at least AMAX_BIG elements (four times the loads in flight: 5.1 -> 3.8 us
// at 17408x256, 9.8 -> 5.5 at 32768x256), 256 below (0.1 us faster at 768x512 and 2048x256); AMAX_BLOCKS
// partial maxima either way
constexpr long AMAX_BIG = 1L << 20;
void launch_amax(const MatsIn& X, long ldx, int K, int r, uint32_t* part, uint32_t* bar, int n, hipStream_t st) {
    if ((long)K * r >= AMAX_BIG)
        k_amax<1024><<<dim3(AMAX_BLOCKS, 1, n), 1024, 0, st>>>(X, ldx, K, r, part, bar);
    else
        k_amax<256><<<dim3(AMAX_BLOCKS, 1, n), 256, 0, st>>>(X, ldx, K, r, part, bar);
}

// word[i * stride] = 0 for i < n (clears wait-error words where no k_amax runs first)
__global__ void k_clear_words(uint32_t* word, int n, int stride) {
    if ((int)threadIdx.x < n) word[(size_t)threadIdx.x * stride] = 0u;
}

// bar[3] |= bar[2]: the column-blocked path runs kcholf once per block, each run clearing bar[2] first, so the
// error of the whole call is kept in bar[3] (cleared at the call's start)
__global__ void k_keep_error(uint32_t* bar) {
    if (threadIdx.x == 0 && bar[2] != 0u) bar[3] = 1u;
}

// Q = Y for a call without polish steps (ns = 0), NaN when the call's Cholesky gave up a wait (as k_nsapply)
__global__ __launch_bounds__(256) void k_copy_out(const MatsIn Ys, long ldy, int K, int r, const MatsOut Outs, long ldo,
                                                  const uint32_t* err) {
    const float* __restrict__ Y = Ys.p[blockIdx.z];
    float* __restrict__ Out = Outs.p[blockIdx.z];
    const bool failed = err[(size_t)blockIdx.z * BAR_STRIDE + 2] != 0u;
    const int r4 = r >> 2;
    for (int e = blockIdx.x * 256 + threadIdx.x; e < K * r4; e += gridDim.x * 256) {
        const int row = e / r4, c4 = e - row * r4;
        float4 v = *reinterpret_cast<const float4*>(Y + (size_t)row * ldy + 4 * c4);
        if (failed) v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
        *reinterpret_cast<float4*>(Out + (size_t)row * ldo + 4 * c4) = v;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Column-blocked path (r > 512, kbig.py:69-95): W = s X[:, j:j+256] for one block, s the power-of-2 scale of all of
// X (from the amax partials of the whole matrix). Exact: s is a power of 2.
// ---------------------------------------------------------------------------------------------------------------
constexpr int BW = 256;   // block width orth.py:19 uses (borth(X, 256)); spanqr_plan_create_borth takes others
__global__ __launch_bounds__(256) void k_scale_block(const float* __restrict__ X, long ldx, int K, int bw,
                                                     const uint32_t* __restrict__ amax_part, float* __restrict__ W) {
    const float sc = block_scale(amax_part);
    const int b4 = bw / 4, n4 = K * b4;
    for (int e = blockIdx.x * 256 + threadIdx.x; e < n4; e += gridDim.x * 256) {
        const int row = e / b4, c4 = e - row * b4;
        float4 v = *reinterpret_cast<const float4*>(X + (size_t)row * ldx + 4 * c4);
        v.x = sc * v.x; v.y = sc * v.y; v.z = sc * v.z; v.w = sc * v.w;
        *reinterpret_cast<float4*>(W + (size_t)row * bw + 4 * c4) = v;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------------------------------
thread_local std::string g_err;
// polls of one bounded wait before the Cholesky gives up on it (spanqr_debug_spin_limit lowers it for the tests of
// the failure path)
uint32_t g_spin_limit = SPIN_LIMIT;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIPCHK(x)                                                                                 \
    do {                                                                                          \
        hipError_t e_ = (x);                                                                      \
        if (e_ != hipSuccess) return fail(SPANQR_EHIP, "%s: %s", #x, hipGetErrorString(e_));      \
    } while (0)

// keeps the caller's current device and restores it on scope exit
struct DeviceGuard {
    int prev = -1;
    bool ok = false;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) == hipSuccess && (prev == dev || hipSetDevice(dev) == hipSuccess)) ok = true;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace

struct spanqr_plan {
    int K = 0, r = 0, device = 0;
    int batch = 1, chol_bmax = 1;   // matrices per call; matrices per Cholesky launch
    size_t lp_stride = 0;           // floats of packed factor per matrix
    int nt = 0, U = 0, NB = 0, S = 0, KS = 0, chol_grid = 0, trsm_q = 0, trsm_rb = 1;   // NB: 32-column blocks
    bool gram_short = false;  // one-launch Gram over upper 32x32 tiles (k_gram32) instead of split Gram + reduction
    int nnp = 0;              // norm partials per matrix the Gram writes (16 per 64x64 tile, or 1 per 32x32 tile)
    int owner_w = OWNER_W;    // tiles per Cholesky owner part at most
    bool trsm_rows = false;   // solve with a wavefront pair per 16 rows (k_trsm_rows) instead of k_trsm
    int solve_rb = 0;         // row blocks per solve workgroup in the Cholesky's launch (0: separate launches)
    int solve_nrb = 0;        // solve workgroups per matrix there
    int solve_wpg = TRSM_NW;  // row blocks per workgroup of the one-wavefront-per-row-block solve
    int solve_q = 0;          // their column blocks per wave (k_trsm's Q), or 0: one wavefront per row block
    int cus = 0;              // the device's compute units
    uint32_t* colcnt = nullptr;   // per matrix: the column counters of the solve in the Cholesky's launch
    size_t bytes = 0;
    char* base = nullptr;
    float *Z = nullptr, *P = nullptr, *G = nullptr, *L = nullptr, *Li = nullptr, *Y0 = nullptr, *Y1 = nullptr;
    float* Lp = nullptr;       // the factor as packed solve operands (store_tile_op's layout), per matrix
    float* scal = nullptr;     // s, nrm0, tau0, nrm1, tau1, nrm2, tau2, barrier error (as float bits)
    float* chscal = nullptr;   // per-launch Cholesky scalars (nrm, tau, err)
    double* npart = nullptr;
    uint32_t* amax_part = nullptr;
    uint32_t* bar = nullptr;   // per matrix: [unused, unused, wait error, ...]
    uint64_t* stamps = nullptr;  // Cholesky phase stamps (profiling): start, then 4 per 32-column step
    uint32_t* flags = nullptr;   // Cholesky dataflow flags and per-workgroup call counters
    hipEvent_t ev[64] = {};    // profiling: one event before and after each kernel of a call
    // column-blocked path (r > 512): the plan of one 256-column block, the K x r dust whose column slices the blocks
    // use, the block buffer W [K, 256], the projection's split partials and its product T [r - 256, 256], the amax
    // partials of the whole X
    spanqr_plan* blk = nullptr;
    int nblk = 0, bw = 0;   // column-blocked plan: blocks of bw columns
    bool reorth = true;     // project and orthonormalise each block a second time (kbig.py:91-92)
    char* bbase = nullptr;
    float *Zb = nullptr, *W = nullptr, *Tp = nullptr, *T = nullptr;
    uint32_t* bamax = nullptr;
    int nev = 0;
    int last_n = 1;             // matrices of the last call enqueued on the plan (spanqr_plan_status reads theirs)
};

namespace {

// Gram split policy: about 512 workgroups over the U upper tiles, at least 4 chunks of 32 rows per split; fixed by
// (K, r) alone so results do not depend on the device.
void split_policy(int K, int U, int* S_out, int* KS_out) {
    int S = (512 + U - 1) / U;
    const int cap = (K + 4 * BK - 1) / (4 * BK);
    if (S > cap) S = cap;
    if (S < 1) S = 1;
    const int KS = ((K + S - 1) / S + BK - 1) / BK * BK;
    *KS_out = KS;
    *S_out = (K + KS - 1) / KS;
}

// Short X with many tiles takes the one-launch Gram (k_gram32): two row splits of KS = ceil(K / 2) rounded up to 32
// rows inside each 32x32-tile workgroup, where that measured faster than the split Gram with its reduction launch
// (768 x 512: 9.3 against 5.5 + 3.5 us and a launch gap; at r <= 384 or K > 1024 the split Gram's parallelism wins).
// Fixed by (K, r) alone, as the split rule is, so results do not depend on the device.
constexpr int GRAM_SHORT_KMAX = 1024, GRAM_SHORT_RMIN = 448;
bool gram_short_rule(int K, int r) { return K <= GRAM_SHORT_KMAX && r >= GRAM_SHORT_RMIN; }
int gram_short_rows(int K) { return ((K + 1) / 2 + BK - 1) / BK * BK; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
// the kernels address 32 rows of a matrix with 32-bit byte offsets (the short Gram's buffer loads)
constexpr long LD_LIMIT = 1L << 24;

int check_mat(const spanqr_plan* p, const float* M, long ld, const char* name) {
    if (M == nullptr) return fail(SPANQR_EINVAL, "%s is null", name);
    if (!aligned16(M)) return fail(SPANQR_EINVAL, "%s must be 16-byte aligned", name);
    if (ld < p->r || (ld & 3) || ld >= LD_LIMIT)
        return fail(SPANQR_EINVAL, "leading dimension of %s (%ld) must be >= r, below 2^24 and a multiple of 4", name,
                    ld);
    return SPANQR_OK;
}

size_t trsm_lds(int r, int rb) { return (size_t)(16 * rb * (r + 4) + TRSM_NW * 16 * 33 + r / CB + 1) * sizeof(float); }

MatsIn mats_in(const float* const* X, int n) {
    MatsIn m{};
    for (int i = 0; i < n; ++i) m.p[i] = X[i];
    return m;
}
MatsOut mats_out(float* const* X, int n) {
    MatsOut m{};
    for (int i = 0; i < n; ++i) m.p[i] = X[i];
    return m;
}
// a plan-owned [K, r] buffer of every matrix (stride K r)
MatsIn buf_in(const spanqr_plan* p, const float* base) {
    MatsIn m{};
    for (int i = 0; i < p->batch; ++i) m.p[i] = base + (size_t)i * p->K * p->r;
    return m;
}
MatsOut buf_out(const spanqr_plan* p, float* base) {
    MatsOut m{};
    for (int i = 0; i < p->batch; ++i) m.p[i] = base + (size_t)i * p->K * p->r;
    return m;
}

// Chunks per Gram stage: two for splits of at most GRAM_DEEP_KS rows (more loads in flight: 0.2-0.5 us faster at
// 128-row splits), one for longer splits (the two-chunk stage measured ~1 us slower at 352-row splits).
constexpr int GRAM_DEEP_KS = 8 * BK;
// The plain Gram reads its operands straight into registers (k_gramr) for splits of at least GRAMR_MIN_KS rows: per
// launch 19.8 -> 18.2 us at 17408x256 and 20.0 -> 18.3 at 8192x384 (352-row splits), 64.8 -> 56.6 at 16384x512,
// 24.3 -> 23.2 at 65536x128; slower for shorter splits (4096x512, 288 rows: 18.0 -> 20.3; 6144x256, 128 rows:
// 8.7 -> 9.9). Its Kahan and scaled forms measured slower than k_gram's at every shape but 32768x256 and are not kept.
constexpr int GRAMR_MIN_KS = 320;

template <int NCH>
void launch_gram_n(const spanqr_plan* p, const MatsIn& A, long lda, dim3 grid, bool scale, bool kahan, hipStream_t st) {
    const int rc = p->r;
    if (kahan && scale)
        k_gram<true, true, false, NCH><<<grid, 512, 0, st>>>(A, lda, p->K, p->nt, p->KS, p->amax_part, p->P, nullptr, 0, 0, rc);
    else if (kahan)
        k_gram<true, false, false, NCH><<<grid, 512, 0, st>>>(A, lda, p->K, p->nt, p->KS, p->amax_part, p->P, nullptr, 0, 0, rc);
    else if (scale)
        k_gram<false, true, false, NCH><<<grid, 512, 0, st>>>(A, lda, p->K, p->nt, p->KS, p->amax_part, p->P, nullptr, 0, 0, rc);
    else
        k_gram<false, false, false, NCH><<<grid, 512, 0, st>>>(A, lda, p->K, p->nt, p->KS, p->amax_part, p->P, nullptr, 0, 0, rc);
}

void launch_gram(const spanqr_plan* p, const MatsIn& A, long lda, int n, bool scale, bool kahan, hipStream_t st) {
    const dim3 grid(p->U, p->S, n);
    if (!kahan && !scale && p->KS >= GRAMR_MIN_KS)
        k_gramr<<<grid, 256, 0, st>>>(A, lda, p->K, p->nt, p->KS, p->P, p->r);
    else if (p->KS <= GRAM_DEEP_KS)
        launch_gram_n<2>(p, A, lda, grid, scale, kahan, st);
    else
        launch_gram_n<1>(p, A, lda, grid, scale, kahan, st);
}

void launch_reduce(const spanqr_plan* p, int mode, float* out, int n, hipStream_t st) {
    const dim3 grid(16, p->U, n);
    if (mode == 0) k_reduce<0><<<grid, 256, 0, st>>>(p->P, p->S, p->nt, p->r, out, p->npart, p->colcnt);
    else k_reduce<1><<<grid, 256, 0, st>>>(p->P, p->S, p->nt, p->r, out, p->npart);
}

template <bool KAHAN, bool SCALE, int MODE>
void launch_gram32_t(const spanqr_plan* p, const MatsIn& A, long lda, int n, hipStream_t st) {
    const int nb = p->r / CB;
    k_gram32<KAHAN, SCALE, MODE><<<dim3(nb * (nb + 1) / 2, 1, n), 512, 0, st>>>(A, lda, p->K, nb, p->KS, p->amax_part,
                                                                              p->G, p->npart, p->r, p->colcnt);
}

// G of a pass (mode 0: G, the norm partials, the next Cholesky's column counters cleared) or D = (I - G) / 2 of a
// polish step (mode 1) into p->G: one launch on a short-X plan, else the split Gram and its reduction. mark() after
// each launch (profiling).
template <class Mark>
int launch_gram_g(const spanqr_plan* p, const MatsIn& A, long lda, int n, bool scale, bool kahan, int mode,
                  hipStream_t st, Mark mark) {
    if (p->gram_short) {
        if (mode == 0) {
            if (kahan && scale) launch_gram32_t<true, true, 0>(p, A, lda, n, st);
            else if (kahan) launch_gram32_t<true, false, 0>(p, A, lda, n, st);
            else if (scale) launch_gram32_t<false, true, 0>(p, A, lda, n, st);
            else launch_gram32_t<false, false, 0>(p, A, lda, n, st);
        } else {
            if (kahan) launch_gram32_t<true, false, 1>(p, A, lda, n, st);
            else launch_gram32_t<false, false, 1>(p, A, lda, n, st);
        }
        return mark();
    }
    launch_gram(p, A, lda, n, scale, kahan, st);
    int rc = mark();
    if (rc) return rc;
    launch_reduce(p, mode, p->G, n, st);
    return mark();
}

// Cholesky of the n matrices in p->G, in launches of at most chol_bmax matrices: plan creation has checked that
// chol_bmax * chol_grid workgroups fit on the device at once, which the flag waits of one launch rely on.
// scal: the first matrix's scalar pair (stride SCAL_STRIDE per matrix) or null.
int launch_chol(spanqr_plan* p, float alpha, float tau, float* scal, hipStream_t st, int nnp, int n,
                bool stamp = false, const float* tau_ptr = nullptr) {
    const size_t r = p->r;
    const size_t lds = chol_lds_bytes(p->r, p->owner_w);
    for (int z0 = 0; z0 < n; z0 += p->chol_bmax) {
        const int nz = (n - z0 < p->chol_bmax) ? n - z0 : p->chol_bmax;
        float* A = p->G + z0 * r * r;
        const double* np = p->npart + (size_t)z0 * nnp;
        float* L = p->L + z0 * r * r;
        float* Li = p->Li + z0 * r * CB;
        float* Lp = p->Lp + z0 * p->lp_stride;
        uint32_t* bar = p->bar + (size_t)z0 * BAR_STRIDE;
        uint32_t* flags = p->flags + (size_t)z0 * FLAG_STRIDE;
        float* sc = scal ? scal + (size_t)z0 * SCAL_STRIDE : nullptr;
        const dim3 grid(p->chol_grid, 1, nz);
        if (stamp)
            k_chol<true><<<grid, 512, lds, st>>>(A, p->r, np, nnp, alpha, tau, L, Li, Lp, bar, flags, sc, p->stamps,
                                                 g_spin_limit, p->owner_w, tau_ptr);
        else
            k_chol<false><<<grid, 512, lds, st>>>(A, p->r, np, nnp, alpha, tau, L, Li, Lp, bar, flags, sc, p->stamps,
                                                  g_spin_limit, p->owner_w, tau_ptr);
        HIPCHK(hipGetLastError());
    }
    return SPANQR_OK;
}

// LDS of the Cholesky's launch with its solve: the larger of the two roles' needs (q = 0: the wavefront-per-row-block
// solve, eight transpose tiles and a word)
size_t fused_lds(int r, int ow, int q, int rb) {
    const size_t a = chol_lds_bytes(r, ow), b = q ? trsm_lds(r, rb) : (TRSM_NW * 16 * 33 + 1) * sizeof(float);
    return a > b ? a : b;
}

// The widest r each solve instantiation runs: Q column blocks per wave cover up to 8 Q blocks of 32 columns
constexpr int trsm_q_max_r(int q) { return 8 * q * CB; }

// The maximum dynamic LDS of a kernel is an attribute of the kernel, shared by every plan that launches it, so each
// instantiation's limit is set once per device to the most any plan can ask of it (the widest r it runs, the widest
// owner parts): a later plan that needs less can then never lower the limit under an earlier plan's launches.
// Limits above the device's per-workgroup maximum are clamped to it (plan creation checks each plan's own need).
template <class F>
hipError_t set_lds_limit(F* kernel, size_t need, int maxsh) {
    const int v = need < (size_t)maxsh ? (int)need : maxsh;
    return hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, v);
}

template <int Q, int RB>
hipError_t trsm_limits(int maxsh) {
    const size_t need = trsm_lds(trsm_q_max_r(Q), RB);
    hipError_t e = set_lds_limit(k_trsm<true, Q, RB>, need, maxsh);
    if (e == hipSuccess) e = set_lds_limit(k_trsm<false, Q, RB>, need, maxsh);
    return e;
}

// the fused instantiations: Q = 1 (r <= 256) with one row block, Q = 2 (r <= 512) with one or two, Q = 4
// (r <= 1024) with one, and the wavefront-per-row-block solve (Q = 0) for r/32 = RB = 2, 4, 6, 8 column blocks
template <int Q, int RB>
hipError_t fused_limits(int maxsh) {
    const int rmax = Q > 0 ? trsm_q_max_r(Q) : RB * CB;
    const size_t need = fused_lds(rmax, OWNER_WMAX, Q, RB);
    hipError_t e = set_lds_limit(k_chol_solve<true, Q, RB>, need, maxsh);
    if (e == hipSuccess) e = set_lds_limit(k_chol_solve<false, Q, RB>, need, maxsh);
    return e;
}

std::mutex g_lds_mu;
bool g_lds_done[64] = {};

// every dynamic-LDS kernel's limit on `device` (current), once per process
int kernel_lds_limits(int device) {
    std::lock_guard<std::mutex> lk(g_lds_mu);
    const bool track = device >= 0 && device < 64;
    if (track && g_lds_done[device]) return SPANQR_OK;
    int maxsh = 0;
    HIPCHK(hipDeviceGetAttribute(&maxsh, hipDeviceAttributeMaxSharedMemoryPerBlock, device));
    hipError_t e = trsm_limits<1, 1>(maxsh);
    if (e == hipSuccess) e = trsm_limits<2, 1>(maxsh);
    if (e == hipSuccess) e = trsm_limits<2, 2>(maxsh);
    if (e == hipSuccess) e = trsm_limits<4, 1>(maxsh);
    if (e == hipSuccess) e = fused_limits<1, 1>(maxsh);
    if (e == hipSuccess) e = fused_limits<2, 1>(maxsh);
    if (e == hipSuccess) e = fused_limits<2, 2>(maxsh);
    if (e == hipSuccess) e = fused_limits<4, 1>(maxsh);
    if (e == hipSuccess) e = fused_limits<0, 2>(maxsh);
    if (e == hipSuccess) e = fused_limits<0, 4>(maxsh);
    if (e == hipSuccess) e = fused_limits<0, 6>(maxsh);
    if (e == hipSuccess) e = fused_limits<0, 8>(maxsh);
    if (e == hipSuccess) e = set_lds_limit(k_chol<true>, chol_lds_bytes(KCH_MAX_R, OWNER_WMAX), maxsh);
    if (e == hipSuccess) e = set_lds_limit(k_chol<false>, chol_lds_bytes(KCH_MAX_R, OWNER_WMAX), maxsh);
    if (e == hipSuccess) e = set_lds_limit(k_nsapply_res<512>, nsr_lds_bytes<512>(), maxsh);
    if (e != hipSuccess) return fail(SPANQR_EHIP, "setting the kernels' LDS limits failed: %s", hipGetErrorString(e));
    if (track) g_lds_done[device] = true;
    return SPANQR_OK;
}

// the dust the pass-1 solve adds: the plan's own Z [K, r], or a column slice of a wider one (row stride ldz)
struct Dust {
    const float* z;
    long ldz;
};

template <int Q, int RB>
void launch_trsm_t(const spanqr_plan* p, const MatsIn& A, long lda, bool pass1, float eps, const Dust& dz,
                   const MatsOut& Y, long ldy, int n, hipStream_t st) {
    const dim3 grid((p->K + 16 * RB - 1) / (16 * RB), 1, n);
    const size_t lds = trsm_lds(p->r, RB);
    if (pass1) k_trsm<true, Q, RB><<<grid, 64 * TRSM_NW, lds, st>>>(A, lda, p->K, p->r, p->amax_part, dz.z, dz.ldz, eps, p->Lp,
                                                           Y, ldy, p->scal);
    else k_trsm<false, Q, RB><<<grid, 64 * TRSM_NW, lds, st>>>(A, lda, p->K, p->r, p->amax_part, dz.z, dz.ldz, eps, p->Lp, Y,
                                                      ldy, p->scal);
}

template <int Q>
void launch_trsm_q(const spanqr_plan* p, const MatsIn& A, long lda, bool pass1, float eps, const Dust& dz,
                   const MatsOut& Y, long ldy, int n, hipStream_t st) {
    if constexpr (Q == 2) {
        if (p->trsm_rb == 2) {
            launch_trsm_t<Q, 2>(p, A, lda, pass1, eps, dz, Y, ldy, n, st);
            return;
        }
    }
    launch_trsm_t<Q, 1>(p, A, lda, pass1, eps, dz, Y, ldy, n, st);
}

template <int NBC>
void launch_trsm_rows(const spanqr_plan* p, const MatsIn& A, long lda, bool pass1, float eps, const Dust& dz,
                      const MatsOut& Y, long ldy, int n, hipStream_t st) {
    const dim3 grid((p->K + 15) / 16, 1, n);
    if (pass1) k_trsm_rows<true, NBC><<<grid, 128, 0, st>>>(A, lda, p->K, p->amax_part, dz.z, dz.ldz, eps, p->Lp, Y,
                                                            ldy, p->scal);
    else k_trsm_rows<false, NBC><<<grid, 128, 0, st>>>(A, lda, p->K, p->amax_part, dz.z, dz.ldz, eps, p->Lp, Y, ldy,
                                                       p->scal);
}

// Y = A L^-T for the n matrices, with the packed factors the plan's Cholesky left in p->Lp
void launch_trsm(const spanqr_plan* p, const MatsIn& A, long lda, bool pass1, float eps, const Dust& dz,
                 const MatsOut& Y, long ldy, int n, hipStream_t st) {
    if (p->trsm_rows) {
        switch (p->r / CB) {
            case 2: launch_trsm_rows<2>(p, A, lda, pass1, eps, dz, Y, ldy, n, st); break;
            case 4: launch_trsm_rows<4>(p, A, lda, pass1, eps, dz, Y, ldy, n, st); break;
            case 6: launch_trsm_rows<6>(p, A, lda, pass1, eps, dz, Y, ldy, n, st); break;
            default: launch_trsm_rows<8>(p, A, lda, pass1, eps, dz, Y, ldy, n, st); break;
        }
        return;
    }
    switch (p->trsm_q) {
        case 1: launch_trsm_q<1>(p, A, lda, pass1, eps, dz, Y, ldy, n, st); break;
        case 2: launch_trsm_q<2>(p, A, lda, pass1, eps, dz, Y, ldy, n, st); break;
        default: launch_trsm_q<4>(p, A, lda, pass1, eps, dz, Y, ldy, n, st); break;
    }
}

template <bool PASS1, int Q, int RB>
void launch_fused_t(dim3 grid, size_t lds, hipStream_t st, const CholArgs& c, const SolveArgs& t) {
    k_chol_solve<PASS1, Q, RB><<<grid, 64 * TRSM_NW, lds, st>>>(c, t);
}

template <bool PASS1>
void launch_fused(int q, int rb, dim3 grid, size_t lds, hipStream_t st, const CholArgs& c, const SolveArgs& t) {
    if (q == 4) {
        launch_fused_t<PASS1, 4, 1>(grid, lds, st, c, t);
        return;
    }
    if (q == 2) {
        if (rb == 2) launch_fused_t<PASS1, 2, 2>(grid, lds, st, c, t);
        else launch_fused_t<PASS1, 2, 1>(grid, lds, st, c, t);
        return;
    }
    if (q == 1) {
        launch_fused_t<PASS1, 1, 1>(grid, lds, st, c, t);
        return;
    }
    switch (rb) {
        case 2: launch_fused_t<PASS1, 0, 2>(grid, lds, st, c, t); break;
        case 4: launch_fused_t<PASS1, 0, 4>(grid, lds, st, c, t); break;
        case 6: launch_fused_t<PASS1, 0, 6>(grid, lds, st, c, t); break;
        default: launch_fused_t<PASS1, 0, 8>(grid, lds, st, c, t); break;
    }
}

// One pass's Cholesky of the n matrices in p->G with the solve Y = A L^-T in the same launches (k_chol_solve), at most
// chol_bmax matrices per launch. The column counters start at zero (k_reduce clears them before every Cholesky).
int launch_chol_solve(spanqr_plan* p, float alpha, float tau, float* scal, hipStream_t st, int nnp, int n,
                      const MatsIn& A, long lda, bool pass1, float eps, const Dust& dz, const MatsOut& Y, long ldy) {
    const size_t r = p->r;
    const int q = p->solve_q;
    const size_t lds = fused_lds(p->r, p->owner_w, q, p->solve_rb);
    for (int z0 = 0; z0 < n; z0 += p->chol_bmax) {
        const int nz = (n - z0 < p->chol_bmax) ? n - z0 : p->chol_bmax;
        CholArgs c;
        c.A = p->G + z0 * r * r;
        c.npart = p->npart + (size_t)z0 * nnp;
        c.L = p->L + z0 * r * r;
        c.Li = p->Li + z0 * r * CB;
        c.Lp = p->Lp + z0 * p->lp_stride;
        c.bar = p->bar + (size_t)z0 * BAR_STRIDE;
        c.flags = p->flags + (size_t)z0 * FLAG_STRIDE;
        c.scal = scal ? scal + (size_t)z0 * SCAL_STRIDE : nullptr;
        c.colcnt = p->colcnt + (size_t)z0 * CC_STRIDE * CH_MAXROW;
        c.alpha = alpha;
        c.tau_rel = tau;
        c.r = p->r;
        c.nnp = nnp;
        c.nz = nz;
        c.grid = p->chol_grid;
        c.ow = p->owner_w;
        c.lim = g_spin_limit;
        SolveArgs t{};
        for (int i = 0; i < nz; ++i) {
            t.A.p[i] = A.p[z0 + i];
            t.Y.p[i] = Y.p[z0 + i];
        }
        t.amax_part = p->amax_part + (size_t)z0 * AMAX_BLOCKS;
        t.Z = dz.z;
        t.scal = p->scal + (size_t)z0 * SCAL_STRIDE;
        t.lda = lda;
        t.ldz = dz.ldz;
        t.ldy = ldy;
        t.eps = eps;
        t.K = p->K;
        t.nrb = p->solve_nrb;
        t.wpg = p->solve_wpg;
        const dim3 grid(nz * (p->chol_grid + p->solve_nrb));
        if (pass1) launch_fused<true>(q, q ? p->solve_rb : p->r / CB, grid, lds, st, c, t);
        else launch_fused<false>(q, q ? p->solve_rb : p->r / CB, grid, lds, st, c, t);
        HIPCHK(hipGetLastError());
    }
    return SPANQR_OK;
}

void launch_nsapply(const spanqr_plan* p, const MatsIn& Y, long ldy, const MatsOut& Out, long ldo, int n,
                    hipStream_t st) {
    // 64-column steps: half the load-then-multiply steps of each workgroup's chain (1-1.5 us faster at 17408x256
    // and 768x512 than 32-column steps, level elsewhere)
    // r % 64 == 32: 32-column steps (the chain over r stays exact: no step past r) and a half-used last column tile
    const dim3 grid((p->K + 31) / 32, (p->r + 63) / 64, n);
    if ((long)grid.x * grid.y * n > 2L * p->cus && p->r % 64 == 0 && p->r <= 512) {
        // two workgroups per CU over the n matrices: G row groups per matrix (a multiple of 8, at most the number of
        // 16-row blocks rounded up)
        const int nslab = p->r / 64, nblk = (p->K + 15) / 16;
        int G = (2 * p->cus / (nslab * n)) / 8 * 8;
        G = std::max(8, std::min(G, (nblk + 7) / 8 * 8));
        if (p->r <= 256)
            k_nsapply_res<256><<<dim3(nslab * G, 1, n), 256, nsr_lds_bytes<256>(), st>>>(Y, ldy, p->K, p->r, p->G,
                                                                                       Out, ldo, p->bar, G);
        else
            k_nsapply_res<512><<<dim3(nslab * G, 1, n), 256, nsr_lds_bytes<512>(), st>>>(Y, ldy, p->K, p->r, p->G,
                                                                                       Out, ldo, p->bar, G);
    } else if ((long)grid.x * grid.y * n <= 2L * p->cus && p->r % 64 == 0) {
        // an even number of steps: 64 columns when r % 128 == 0, else 32
        if (p->r % 128 == 0)
            k_nsapply_pipe<64><<<grid, 256, 0, st>>>(Y, ldy, p->K, p->r, p->G, Out, ldo, p->bar);
        else
            k_nsapply_pipe<32><<<grid, 256, 0, st>>>(Y, ldy, p->K, p->r, p->G, Out, ldo, p->bar);
    } else if (p->r % 64 == 0)
        k_nsapply<false, 64><<<grid, 256, 0, st>>>(Y, ldy, p->K, p->r, p->G, Out, ldo, nullptr, 0, 0, p->bar);
    else
        k_nsapply<false, 32><<<grid, 256, 0, st>>>(Y, ldy, p->K, p->r, p->G, Out, ldo, nullptr, 0, 0, p->bar);
}


// The whole call on one stream for n matrices: amax, 3 x {gram, reduce, chol, trsm}, ns x {gram, reduce, nsapply},
// each kernel launched once for all n (the Cholesky in groups of chol_bmax). With rec, an event is recorded after
// every kernel (profiling).
int enqueue_orth(spanqr_plan* p, int n, const MatsIn& X, long ldx, const MatsOut& Q, long ldq, float eps, float alpha,
                 float tau, int ns, hipStream_t st, bool rec, Dust dz = Dust{nullptr, 0}) {
    if (dz.z == nullptr) dz = Dust{p->Z, p->r};
    p->last_n = n;
    int rc;
    auto mark = [&]() -> int {
        if (rec) {
            HIPCHK(hipEventRecord(p->ev[p->nev], st));
            ++p->nev;
        }
        return SPANQR_OK;
    };
    launch_amax(X, ldx, p->K, p->r, p->amax_part, p->bar, n, st);
    if ((rc = mark())) return rc;
    const MatsIn bin[2] = {buf_in(p, p->Y0), buf_in(p, p->Y1)};
    const MatsOut bout[2] = {buf_out(p, p->Y0), buf_out(p, p->Y1)};
    const MatsIn* in = &X;
    long ldin = ldx;
    int cur = 0;
    for (int pass = 0; pass < 3; ++pass) {
        if ((rc = launch_gram_g(p, *in, ldin, n, pass == 0, pass == 0, 0, st, mark))) return rc;
        // the solve in the Cholesky's launch when every workgroup of the launch fits on the device at once (one per
        // CU); a larger batch runs them as separate launches, where the solve keeps its own, smaller LDS
        if (p->solve_rb > 0 && n * (p->chol_grid + p->solve_nrb) <= p->cus) {
            if ((rc = launch_chol_solve(p, alpha, tau, p->scal + 1 + 2 * pass, st, p->nnp, n, *in, ldin, pass == 0,
                                        eps, dz, bout[cur], p->r)))
                return rc;
            if ((rc = mark())) return rc;
        } else {
            if ((rc = launch_chol(p, alpha, tau, p->scal + 1 + 2 * pass, st, p->nnp, n))) return rc;
            if ((rc = mark())) return rc;
            launch_trsm(p, *in, ldin, pass == 0, eps, dz, bout[cur], p->r, n, st);
            if ((rc = mark())) return rc;
        }
        in = &bin[cur];
        ldin = p->r;
        cur ^= 1;
    }
    for (int i = 0; i < ns; ++i) {
        if ((rc = launch_gram_g(p, *in, ldin, n, false, i == ns - 1, 1, st, mark))) return rc;
        if (i == ns - 1) {
            launch_nsapply(p, *in, ldin, Q, ldq, n, st);
        } else {
            launch_nsapply(p, *in, ldin, bout[cur], p->r, n, st);
            in = &bin[cur];
            cur ^= 1;
        }
        if ((rc = mark())) return rc;
    }
    if (ns == 0) {
        const int blocks = (p->K * (p->r / 4) + 255) / 256 < 1024 ? (p->K * (p->r / 4) + 255) / 256 : 1024;
        k_copy_out<<<dim3(blocks, 1, n), 256, 0, st>>>(*in, ldin, p->K, p->r, Q, ldq, p->bar);
    }
    HIPCHK(hipGetLastError());
    return SPANQR_OK;
}

}  // namespace

extern "C" {

const char* spanqr_last_error(void) { return g_err.c_str(); }

int spanqr_dust_host(int K, int r, float* Z) {
    if (K <= 0 || r <= 0 || Z == nullptr) return fail(SPANQR_EINVAL, "dust: bad arguments");
    const uint64_t key = mix64(20261018ull);
    double* n2 = (double*)calloc((size_t)r, sizeof(double));
    if (!n2) return fail(SPANQR_ENOMEM, "dust: out of host memory");
    for (int k = 0; k < K; ++k)
        for (int c = 0; c < r; ++c) {
            const uint64_t n = (uint64_t)k * (uint64_t)r + (uint64_t)c;
            uint64_t S = 0;
            for (uint64_t j = 0; j < 6; ++j) {
                const uint64_t wv = mix64(key + (6 * n + j + 1) * 0x9E3779B97F4A7C15ull);
                S += (wv & 0xffffffffull) + (wv >> 32);
            }
            const float z = (float)ldexp((double)((int64_t)S - (int64_t)6 * 4294967295ll), -32);
            Z[(size_t)k * r + c] = z;
            n2[c] += (double)z * (double)z;
        }
    for (int c = 0; c < r; ++c) n2[c] = sqrt(n2[c]);
    for (int k = 0; k < K; ++k)
        for (int c = 0; c < r; ++c) Z[(size_t)k * r + c] = (float)((double)Z[(size_t)k * r + c] / n2[c]);
    free(n2);
    return SPANQR_OK;
}

static int check_shape(int K, int r, bool blocked_ok = false) {
    const bool blocked = blocked_ok && r > 512 && r <= SPANQR_MAX_R && (r % BW) == 0;
    if (!blocked && (r < 32 || r > KCH_MAX_R || (r % 32) != 0))
        return fail(SPANQR_EINVAL, blocked_ok ? "r = %d: must be a multiple of 32 in [32, 1024] or of 256 up to 4096"
                                              : "r = %d: must be a multiple of 32 in [32, 1024]", r);
    if (K < r) return fail(SPANQR_EINVAL, "K = %d < r = %d", K, r);
    if ((long)K * r >= (1L << 30)) return fail(SPANQR_EINVAL, "K * r too large");
    return SPANQR_OK;
}

namespace {

size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

// Shape-derived fields of a kcholf plan (r <= 512): the Gram's split rule, the Cholesky's grid, the solve variant.
void plan_shape(spanqr_plan* p, int K, int r, int batch) {
    p->K = K; p->r = r; p->batch = batch;
    p->nt = (r + TB - 1) / TB; p->U = p->nt * (p->nt + 1) / 2; p->NB = r / CB;
    p->gram_short = gram_short_rule(K, r);
    if (p->gram_short) {
        p->KS = gram_short_rows(K);
        p->S = (K + p->KS - 1) / p->KS;
        p->nnp = p->NB * (p->NB + 1) / 2;
    } else {
        split_policy(K, p->U, &p->S, &p->KS);
        p->nnp = 16 * p->U;
    }
    p->owner_w = OWNER_W;
    p->chol_grid = chol_workgroups(r / CB, p->owner_w);     // workgroup 0 + the parts of tile rows 4..r/32-1
    p->trsm_q = trsm_q_for(r / CB);
    // solve: RB row blocks of 16 per workgroup; one block while that leaves fewer than ~2 workgroups per CU (and
    // always one with four column blocks per wavefront, r > 512)
    p->trsm_rb = ((K + 15) / 16 >= 1024 && p->trsm_q <= 2) ? 2 : 1;
    // a wavefront pair per 16 rows once there are enough rows to occupy the SIMDs (the chain over r/32 blocks is
    // long; the measured crossover at r = 256 lies near K = 8192-10240); below that, k_trsm splits each row block's
    // columns over eight waves
    p->trsm_rows = r <= 256 && K >= 9216 && (r / CB) % 2 == 0;   // instantiated for 2, 4, 6, 8 column blocks
    p->lp_stride = (size_t)(r / CB) * (r / CB + 1) / 2 * CB * CB;
}

// Per-device set-up of a kcholf plan's kernels: the dynamic LDS limits of the solve and the Cholesky, and the
// co-residency check that the Cholesky's flag waits rely on; sets chol_bmax (at most batch).
int plan_device_setup(spanqr_plan* p, int device) {
    const int r = p->r;
    int rc = kernel_lds_limits(device);
    if (rc != SPANQR_OK) return rc;
    {
        const size_t need = trsm_lds(r, p->trsm_rb);
        int maxsh = 0;
        HIPCHK(hipDeviceGetAttribute(&maxsh, hipDeviceAttributeMaxSharedMemoryPerBlock, device));
        if ((size_t)maxsh < need)
            return fail(SPANQR_EHIP, "the solve needs %zu bytes of LDS per workgroup, device allows %d", need, maxsh);
    }
    int occ = 0, cus = 0;
    HIPCHK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
    p->cus = cus;
    // The owner part width: OWNER_W for one matrix; for a batch, the narrowest of 6, 8, 12 and 16 tiles that runs
    // the batch's Cholesky in the fewest launches (each launch needs all its workgroups resident at once, within
    // three quarters of the device: the margin leaves room for work of other streams)
    {
        const int widths[] = {OWNER_W, 8, 12, OWNER_WMAX};
        int best_w = 0, best_n = 1 << 30, best_occ = 0;
        for (int w : widths) {
            if (p->batch == 1 && w != OWNER_W) break;
            int o = 0;
            HIPCHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, (const void*)k_chol<true>, 512, chol_lds_bytes(r, w)));
            const int grid = chol_workgroups(r / CB, w);
            if (o * cus < grid) continue;
            int bmax = (o * cus * 3 / 4) / grid;
            if (bmax < 1) bmax = 1;
            const int launches = (p->batch + bmax - 1) / bmax;
            if (launches < best_n) {
                best_n = launches;
                best_w = w;
                best_occ = o;
            }
        }
        if (best_w == 0)
            return fail(SPANQR_EHIP, "the Cholesky needs %d co-resident workgroups, device holds too few",
                        chol_workgroups(r / CB, OWNER_WMAX));
        p->owner_w = best_w;
        p->chol_grid = chol_workgroups(r / CB, best_w);
        occ = best_occ;
    }
    // a batch's launch takes at most three quarters of the device's resident capacity: the flag waits need every
    // workgroup of a launch resident at once, and the margin leaves room for work of other streams
    p->chol_bmax = (occ * cus * 3 / 4) / p->chol_grid;
    if (p->chol_bmax < 1) p->chol_bmax = 1;
    if (p->chol_bmax > p->batch) p->chol_bmax = p->batch;
    // The solve in the Cholesky's launch: enough rows per workgroup that one matrix's solve workgroups are resident
    // beside its Cholesky (one workgroup per CU: the launch's LDS is the Cholesky's); otherwise separate launches.
    // Up to one row block per CU: k_trsm's structure (eight wavefronts share a row block's column blocks); taller X at
    // r <= 256: one wavefront per row block (eight per workgroup); taller X at r > 256: k_trsm with two row blocks.
    p->solve_rb = 0;
    p->solve_nrb = 0;
    p->solve_q = 0;
    {
        int maxsh = 0;
        HIPCHK(hipDeviceGetAttribute(&maxsh, hipDeviceAttributeMaxSharedMemoryPerBlock, device));
        const int avail = cus - p->chol_grid;
        const int rowblocks = (p->K + 15) / 16;
        int q = trsm_q_for(r / CB), rb = 1, nwg = rowblocks, wpg = TRSM_NW;
        if (rowblocks > avail) {
            if (q == 4 || (r <= 256 && (r / CB) % 2 != 0)) {
                // separate launches: the one-wavefront solve is built for an even number of column blocks, and
                // four column blocks per wavefront for one row block per workgroup only
                nwg = avail + 1;
            } else if (r <= 256) {
                // one wavefront per row block, as few per workgroup (and so per CU) as the free CUs allow
                q = 0;
                wpg = (rowblocks + avail - 1) / avail;
                if (wpg > TRSM_NW) wpg = TRSM_NW;
                nwg = (rowblocks + wpg - 1) / wpg;
            } else {
                rb = 2;
                nwg = (rowblocks + 1) / 2;
            }
        }
        const size_t lds = fused_lds(r, p->owner_w, q, rb);
        if (nwg <= avail && lds <= (size_t)maxsh) {
            p->solve_q = q;
            p->solve_rb = rb;
            p->solve_nrb = nwg;
            p->solve_wpg = wpg;
        }
    }
    return SPANQR_OK;
}

// Workspace of a kcholf plan, 256-byte aligned buffers in this order: Z first (the dust: uploaded or generated; the
// rest starts zeroed), then the Gram partials, G, L, Li, Lp, Y0, Y1, scalars, Cholesky scalars, norm partials, amax
// partials, error words, stamps, flags. Assigns the pointers from base (nullptr: sizes only); returns the bytes.
size_t plan_layout(spanqr_plan* p, char* base) {
    const size_t B = (size_t)p->batch, K = p->K, r = p->r;
    const size_t nKr = K * r * sizeof(float);
    const size_t sz[] = {
        al256(nKr),                                             // Z
        al256(B * p->S * p->U * TB * TB * sizeof(float)),       // P
        al256(B * r * r * sizeof(float)),                       // G
        al256(B * r * r * sizeof(float)),                       // L
        al256(B * r * CB * sizeof(float)),                      // Li
        al256(B * p->lp_stride * sizeof(float)),                // Lp
        al256(B * nKr), al256(B * nKr),                         // Y0, Y1
        al256(B * SCAL_STRIDE * sizeof(float)),                 // scal
        al256(B * SCAL_STRIDE * sizeof(float)),                 // chscal
        al256(B * p->nnp * sizeof(double)),                     // npart
        al256(B * AMAX_BLOCKS * sizeof(uint32_t)),              // amax_part
        al256(B * BAR_STRIDE * sizeof(uint32_t)),               // bar
        al256((24 * CH_MAXROW + 2) * sizeof(uint64_t)),          // stamps
        al256(B * FLAG_STRIDE * sizeof(uint32_t)),              // flags
        al256(B * CC_STRIDE * CH_MAXROW * sizeof(uint32_t)),    // colcnt
    };
    void** ptrs[] = {(void**)&p->Z, (void**)&p->P, (void**)&p->G, (void**)&p->L, (void**)&p->Li, (void**)&p->Lp,
                     (void**)&p->Y0, (void**)&p->Y1, (void**)&p->scal, (void**)&p->chscal, (void**)&p->npart,
                     (void**)&p->amax_part, (void**)&p->bar, (void**)&p->stamps, (void**)&p->flags,
                     (void**)&p->colcnt};
    size_t off = 0;
    for (size_t i = 0; i < sizeof(sz) / sizeof(sz[0]); ++i) {
        if (base) *ptrs[i] = base + off;
        off += sz[i];
    }
    return off;
}

}  // namespace

namespace {

// 64x64 tiles of a projection's P^T C, P with j columns and C with bw (the last tile row and column half used where
// either is an odd multiple of 32); the split rule takes this count
int proj_tiles(int j, int bw) { return ((j + TB - 1) / TB) * ((bw + TB - 1) / TB); }

// Column-blocked plan: a bw-column block plan plus the blocked path's own buffers (no Gram or Cholesky of its own).
int create_blocked(int K, int r, int bw, bool reorth, int device, spanqr_plan** out) {
    spanqr_plan* p = new spanqr_plan;
    p->K = K; p->r = r; p->device = device; p->batch = 1; p->nblk = r / bw; p->bw = bw; p->reorth = reorth;
    int rc = spanqr_plan_create_batched(K, bw, 1, device, &p->blk);
    if (rc != SPANQR_OK) {
        delete p;
        return rc;
    }
    size_t maxp = 0;   // split partials of the largest projection (U = (j / 64) (bw / 64) tiles for j = r - bw)
    for (int jb = 1; jb < p->nblk; ++jb) {
        int S = 0, KS = 0;
        const int U = proj_tiles(bw * jb, bw);
        split_policy(K, U, &S, &KS);
        if ((size_t)S * U > maxp) maxp = (size_t)S * U;
    }
    auto al = [](size_t n) { return (n + 255) & ~(size_t)255; };
    const size_t sz_Z = al((size_t)K * r * sizeof(float)), sz_W = al((size_t)K * bw * sizeof(float));
    const size_t sz_Tp = al(maxp * TB * TB * sizeof(float)), sz_T = al((size_t)r * bw * sizeof(float));
    const size_t sz_am = al(AMAX_BLOCKS * sizeof(uint32_t));
    const size_t bytes = sz_Z + sz_W + sz_Tp + sz_T + sz_am;
    DeviceGuard dg(device);
    if (hipMalloc((void**)&p->bbase, bytes) != hipSuccess) {
        spanqr_plan_destroy(p->blk);
        delete p;
        return fail(SPANQR_ENOMEM, "workspace allocation of %zu bytes failed", bytes);
    }
    p->bytes = bytes + p->blk->bytes;
    char* c = p->bbase;
    p->Zb = (float*)c; c += sz_Z;
    p->W = (float*)c; c += sz_W;
    p->Tp = (float*)c; c += sz_Tp;
    p->T = (float*)c; c += sz_T;
    p->bamax = (uint32_t*)c; c += sz_am;
    float* hz = (float*)malloc((size_t)K * r * sizeof(float));
    rc = hz ? spanqr_dust_host(K, r, hz) : fail(SPANQR_ENOMEM, "host dust buffer");
    if (rc == SPANQR_OK && (hipMemcpy(p->Zb, hz, (size_t)K * r * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
                            hipDeviceSynchronize() != hipSuccess))
        rc = fail(SPANQR_EHIP, "plan upload failed");
    free(hz);
    if (rc != SPANQR_OK) {
        (void)hipFree(p->bbase);
        spanqr_plan_destroy(p->blk);
        delete p;
        return rc;
    }
    *out = p;
    return SPANQR_OK;
}

// Out = Cin - P (P^T Cin) for P = the j leading columns of Q (row stride ldq) and Cin [K, bw] (row stride ldc): the
// projection of kbig.py:88-89. P^T Cin is a split-K product (fp32 MFMA chains per split, fp64 across splits in split
// order, tri.py's Gram rule for the split count), then one MFMA chain per element of P T, subtracted once.
void project(const spanqr_plan* p, const float* Q, long ldq, int j, const float* Cin, long ldc, float* Out,
             hipStream_t st) {
    const int BW = p->bw, ntb = (BW + TB - 1) / TB;
    const int U = proj_tiles(j, BW);
    int S = 0, KS = 0;
    split_policy(p->K, U, &S, &KS);
    const MatsIn P = mats_in(&Q, 1);
    if (KS <= GRAM_DEEP_KS)
        k_gram<false, false, true, 2><<<dim3(U, S), 512, 0, st>>>(P, ldq, p->K, 0, KS, p->bamax, p->Tp, Cin, ldc, ntb,
                                                                 j, BW);
    else
        k_gram<false, false, true, 1><<<dim3(U, S), 512, 0, st>>>(P, ldq, p->K, 0, KS, p->bamax, p->Tp, Cin, ldc, ntb,
                                                                 j, BW);
    k_reduce<2><<<dim3(16, U), 256, 0, st>>>(p->Tp, S, ntb, BW, p->T, nullptr);
    // the chain over P's j columns in 64-column steps, or 32 where j is an odd multiple of 32 (no step past j)
    const dim3 ag((p->K + 31) / 32, ntb);
    if (j % 64 == 0)
        k_nsapply<true, 64><<<ag, 256, 0, st>>>(P, ldq, p->K, j, p->T, mats_out(&Out, 1), BW, Cin, ldc, BW);
    else
        k_nsapply<true, 32><<<ag, 256, 0, st>>>(P, ldq, p->K, j, p->T, mats_out(&Out, 1), BW, Cin, ldc, BW);
}

// borth (kbig.py:69-95, BCGS2 over bw-column blocks; orth.py:18-19 calls it with 256): per block, W = s X_blk,
// projected twice against the finished blocks, orthonormalised by the full kcholf call with the block's slice of the
// K x r dust; with reorth, projected once more and orthonormalised again. Each block's result goes straight into its
// columns of Q.
int enqueue_borth(spanqr_plan* p, const float* X, long ldx, float* Q, long ldq, float eps, float alpha, float tau,
                  int ns, hipStream_t st) {
    const int K = p->K, BW = p->bw;
    p->last_n = 1;
    k_clear_words<<<1, 64, 0, st>>>(p->blk->bar + 3, 1, BAR_STRIDE);
    launch_amax(mats_in(&X, 1), ldx, K, p->r, p->bamax, nullptr, 1, st);
    const int sgrid = (K * (BW / 4) + 255) / 256 < 1024 ? (K * (BW / 4) + 255) / 256 : 1024;
    int rc;
    for (int jb = 0; jb < p->nblk; ++jb) {
        const int j = BW * jb;
        float* Qj = Q + j;
        const float* Wc = p->W;
        const Dust dz{p->Zb + j, p->r};
        k_scale_block<<<sgrid, 256, 0, st>>>(X + j, ldx, K, BW, p->bamax, p->W);
        if (j > 0) {
            project(p, Q, ldq, j, p->W, BW, p->W, st);
            project(p, Q, ldq, j, p->W, BW, p->W, st);
        }
        if ((rc = enqueue_orth(p->blk, 1, mats_in(&Wc, 1), BW, mats_out(&Qj, 1), ldq, eps, alpha, tau, ns, st, false,
                               dz)))
            return rc;
        k_keep_error<<<1, 64, 0, st>>>(p->blk->bar);
        if (j > 0 && p->reorth) {
            project(p, Q, ldq, j, Qj, ldq, p->W, st);
            if ((rc = enqueue_orth(p->blk, 1, mats_in(&Wc, 1), BW, mats_out(&Qj, 1), ldq, eps, alpha, tau, ns, st,
                                   false, dz)))
                return rc;
            k_keep_error<<<1, 64, 0, st>>>(p->blk->bar);
        }
    }
    HIPCHK(hipGetLastError());
    return SPANQR_OK;
}

}  // namespace

int spanqr_split_rows(int K, int r) {
    const int rc = check_shape(K, r);
    if (rc != SPANQR_OK) return rc;
    spanqr_plan p;
    plan_shape(&p, K, r, 1);
    return p.KS;
}

int spanqr_norm_partials(int K, int r) {
    const int rc = check_shape(K, r);
    if (rc != SPANQR_OK) return rc;
    spanqr_plan p;
    plan_shape(&p, K, r, 1);
    return p.nnp;
}

int spanqr_plan_create(int K, int r, int device, spanqr_plan** out) {
    if (out == nullptr) return fail(SPANQR_EINVAL, "out is null");
    *out = nullptr;
    const int shape_rc = check_shape(K, r, true);
    if (shape_rc != SPANQR_OK) return shape_rc;
    // orth.py:18-19: above 512 columns, a multiple of 256 goes through borth over 256-column blocks
    if (r > 512 && r % BW == 0) return create_blocked(K, r, BW, true, device, out);
    return spanqr_plan_create_batched(K, r, 1, device, out);
}

int spanqr_plan_create_borth(int K, int r, int b, int reorth, int device, spanqr_plan** out) {
    if (out == nullptr) return fail(SPANQR_EINVAL, "out is null");
    *out = nullptr;
    if (b < CB || b > KCH_MAX_R || b % CB != 0)
        return fail(SPANQR_EINVAL, "b = %d: must be a multiple of 32 in [32, %d]", b, KCH_MAX_R);
    if (r <= b || r % b != 0 || r > SPANQR_MAX_R)
        return fail(SPANQR_EINVAL, "r = %d: must be a multiple of b = %d above it, at most %d", r, b, SPANQR_MAX_R);
    if (K < r) return fail(SPANQR_EINVAL, "K = %d < r = %d", K, r);
    if ((long)K * r >= (1L << 30)) return fail(SPANQR_EINVAL, "K * r too large");
    return create_blocked(K, r, b, reorth != 0, device, out);
}

int spanqr_plan_create_batched(int K, int r, int batch, int device, spanqr_plan** out) {
    if (out == nullptr) return fail(SPANQR_EINVAL, "out is null");
    *out = nullptr;
    const int shape_rc = check_shape(K, r);   // kcholf at full width
    if (shape_rc != SPANQR_OK) return shape_rc;
    if (batch < 1 || batch > SPANQR_MAX_BATCH)
        return fail(SPANQR_EINVAL, "batch = %d: must be in [1, %d]", batch, SPANQR_MAX_BATCH);
    DeviceGuard dg(device);
    if (!dg.ok) return fail(SPANQR_EHIP, "cannot select HIP device %d", device);
    spanqr_plan* p = new spanqr_plan;
    p->device = device;
    plan_shape(p, K, r, batch);
    int rc = plan_device_setup(p, device);
    if (rc != SPANQR_OK) {
        delete p;
        return rc;
    }
    p->bytes = plan_layout(p, nullptr);
    if (hipMalloc((void**)&p->base, p->bytes) != hipSuccess) {
        const size_t nb = p->bytes;
        delete p;
        return fail(SPANQR_ENOMEM, "workspace allocation of %zu bytes failed", nb);
    }
    plan_layout(p, p->base);
    const size_t nKr = (size_t)K * r * sizeof(float);
    float* hz = (float*)malloc(nKr);
    rc = hz ? spanqr_dust_host(K, r, hz) : fail(SPANQR_ENOMEM, "host dust buffer");
    if (rc == SPANQR_OK) {
        if (hipMemcpy(p->Z, hz, nKr, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemset(p->base + al256(nKr), 0, p->bytes - al256(nKr)) != hipSuccess ||   // all but Z
            hipDeviceSynchronize() != hipSuccess)
            rc = fail(SPANQR_EHIP, "plan upload failed");
    }
    free(hz);
    if (rc != SPANQR_OK) {
        (void)hipFree(p->base);
        delete p;
        return rc;
    }
    *out = p;
    return SPANQR_OK;
}

void spanqr_plan_destroy(spanqr_plan* p) {
    if (!p) return;
    DeviceGuard dg(p->device);
    (void)hipDeviceSynchronize();
    if (p->blk) {
        spanqr_plan_destroy(p->blk);
        (void)hipFree(p->bbase);
        delete p;
        return;
    }
    for (int i = 0; i < 64; ++i)
        if (p->ev[i]) (void)hipEventDestroy(p->ev[i]);
    (void)hipFree(p->base);
    delete p;
}

long spanqr_plan_query(const spanqr_plan* p, int what) {
    if (!p) return -1;
    switch (what) {
        case SPANQR_Q_K: return p->K;
        case SPANQR_Q_R: return p->r;
        case SPANQR_Q_SPLITS: return p->blk ? p->blk->S : p->S;
        case SPANQR_Q_SPLIT_ROWS: return p->blk ? p->blk->KS : p->KS;
        case SPANQR_Q_CHOL_GRID: return p->blk ? p->blk->chol_grid : p->chol_grid;
        case SPANQR_Q_WORKSPACE_MB: return (long)((p->bytes + (1u << 20) - 1) >> 20);
        case SPANQR_Q_DEVICE: return p->device;
        case SPANQR_Q_BATCH: return p->batch;
        case SPANQR_Q_CHOL_BATCH: return p->blk ? p->blk->chol_bmax : p->chol_bmax;
        case SPANQR_Q_BLOCKS: return p->nblk;
        case SPANQR_Q_BLOCK_WIDTH: return p->bw;
        case SPANQR_Q_NORM_PARTIALS: return p->blk ? p->blk->nnp : p->nnp;
        case SPANQR_Q_SOLVE_ROWS: {
            const spanqr_plan* q = p->blk ? p->blk : p;
            return q->solve_rb == 0 ? 0 : (q->solve_q == 0 ? 16L * q->solve_wpg : 16L * q->solve_rb);
        }
        default: return -1;
    }
}

int spanqr_orth_f32(spanqr_plan* p, const float* X, long ldx, float* Q, long ldq, float eps, float alpha, float tau,
                    int ns, void* stream) {
    if (!p) return fail(SPANQR_EINVAL, "plan is null");
    int rc = check_mat(p, X, ldx, "X");
    if (rc) return rc;
    if ((rc = check_mat(p, Q, ldq, "Q"))) return rc;
    if (ns < 0) return fail(SPANQR_EINVAL, "ns = %d < 0", ns);
    DeviceGuard dg(p->device);
    if (!dg.ok) return fail(SPANQR_EHIP, "cannot select HIP device %d", p->device);
    if (p->blk) return enqueue_borth(p, X, ldx, Q, ldq, eps, alpha, tau, ns, (hipStream_t)stream);
    return enqueue_orth(p, 1, mats_in(&X, 1), ldx, mats_out(&Q, 1), ldq, eps, alpha, tau, ns, (hipStream_t)stream,
                        false);
}

int spanqr_orth_batched_f32(spanqr_plan* p, int n, const float* const* X, long ldx, float* const* Q, long ldq,
                            float eps, float alpha, float tau, int ns, void* stream) {
    if (!p) return fail(SPANQR_EINVAL, "plan is null");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    if (n < 1 || n > p->batch) return fail(SPANQR_EINVAL, "n = %d: must be in [1, %d] (the plan's batch)", n, p->batch);
    if (!X || !Q) return fail(SPANQR_EINVAL, "pointer arrays must not be null");
    int rc;
    char name[32];
    for (int i = 0; i < n; ++i) {
        snprintf(name, sizeof name, "X[%d]", i);
        if ((rc = check_mat(p, X[i], ldx, name))) return rc;
        snprintf(name, sizeof name, "Q[%d]", i);
        if ((rc = check_mat(p, Q[i], ldq, name))) return rc;
    }
    if (ns < 0) return fail(SPANQR_EINVAL, "ns = %d < 0", ns);
    DeviceGuard dg(p->device);
    if (!dg.ok) return fail(SPANQR_EHIP, "cannot select HIP device %d", p->device);
    return enqueue_orth(p, n, mats_in(X, n), ldx, mats_out(Q, n), ldq, eps, alpha, tau, ns, (hipStream_t)stream,
                        false);
}

int spanqr_profile_orth(spanqr_plan* p, const float* X, long ldx, float* Q, long ldq, float eps, float alpha,
                        float tau, int ns, void* stream, float* ms, int max_n, int* n_out) {
    if (!p || !ms || !n_out) return fail(SPANQR_EINVAL, "null argument");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    int rc = check_mat(p, X, ldx, "X");
    if (rc) return rc;
    if ((rc = check_mat(p, Q, ldq, "Q"))) return rc;
    if (ns < 0 || 1 + 12 + 3 * ns > 63) return fail(SPANQR_EINVAL, "ns = %d out of range for profiling", ns);
    DeviceGuard dg(p->device);
    hipStream_t st = (hipStream_t)stream;
    for (int i = 0; i < 64; ++i)
        if (!p->ev[i]) HIPCHK(hipEventCreate(&p->ev[i]));
    HIPCHK(hipEventRecord(p->ev[0], st));
    p->nev = 1;
    if ((rc = enqueue_orth(p, 1, mats_in(&X, 1), ldx, mats_out(&Q, 1), ldq, eps, alpha, tau, ns, st, true))) return rc;
    HIPCHK(hipEventSynchronize(p->ev[p->nev - 1]));
    const int n = p->nev - 1 < max_n ? p->nev - 1 : max_n;
    for (int i = 0; i < n; ++i) HIPCHK(hipEventElapsedTime(&ms[i], p->ev[i], p->ev[i + 1]));
    *n_out = n;
    return SPANQR_OK;
}

int spanqr_profile_kernel(spanqr_plan* p, int which, int reps, float* avg_ms, void* stream) {
    if (!p || !avg_ms) return fail(SPANQR_EINVAL, "null argument");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    if (reps < 1 || reps > 100000) return fail(SPANQR_EINVAL, "reps = %d out of range", reps);
    if (which < SPANQR_K_AMAX || which > SPANQR_K_CHOL_SOLVE) return fail(SPANQR_EINVAL, "unknown kernel %d", which);
    if ((which == SPANQR_K_CHOL_SOLVE_PASS1 || which == SPANQR_K_CHOL_SOLVE) && p->solve_rb == 0)
        return fail(SPANQR_EINVAL, "this plan runs the Cholesky and the solve in separate launches");
    if (which == SPANQR_K_REDUCE && p->gram_short)
        return fail(SPANQR_EINVAL, "this plan's Gram reduces its splits in the same launch");
    DeviceGuard dg(p->device);
    if (!dg.ok) return fail(SPANQR_EHIP, "cannot select HIP device %d", p->device);
    hipStream_t st = (hipStream_t)stream;
    for (int i = 0; i < 2; ++i)
        if (!p->ev[i]) HIPCHK(hipEventCreate(&p->ev[i]));
    const int r = p->r;
    const MatsIn y0 = buf_in(p, p->Y0);
    const MatsOut y1 = buf_out(p, p->Y1);
    auto launch = [&]() -> int {
        switch (which) {
            case SPANQR_K_AMAX: launch_amax(y0, r, p->K, r, p->amax_part, nullptr, 1, st); break;
            case SPANQR_K_GRAM_PASS1:
                if (p->gram_short) launch_gram32_t<true, true, 0>(p, y0, r, 1, st);
                else launch_gram(p, y0, r, 1, true, true, st);
                break;
            case SPANQR_K_GRAM:
                if (p->gram_short) launch_gram32_t<false, false, 0>(p, y0, r, 1, st);
                else launch_gram(p, y0, r, 1, false, false, st);
                break;
            case SPANQR_K_REDUCE: launch_reduce(p, 0, p->G, 1, st); break;
            case SPANQR_K_CHOL: return launch_chol(p, 1e-7f, 1e-8f, p->scal + 1, st, p->nnp, 1);
            case SPANQR_K_TRSM_PASS1: launch_trsm(p, y0, r, true, 5e-7f, Dust{p->Z, r}, y1, r, 1, st); break;
            case SPANQR_K_TRSM: launch_trsm(p, y0, r, false, 0.0f, Dust{p->Z, r}, y1, r, 1, st); break;
            case SPANQR_K_NS_APPLY: launch_nsapply(p, y0, r, y1, r, 1, st); break;
        }
        return SPANQR_OK;
    };
    int rc;
    if (which == SPANQR_K_CHOL_SOLVE_PASS1 || which == SPANQR_K_CHOL_SOLVE) {
        // each launch needs its column counters at zero: cleared by a small kernel outside the timed pair of events
        const bool p1 = which == SPANQR_K_CHOL_SOLVE_PASS1;
        double total = 0.0;
        for (int i = 0; i <= reps; ++i) {
            k_clear_words<<<1, 64, 0, st>>>(p->colcnt, CH_MAXROW, CC_STRIDE);
            HIPCHK(hipEventRecord(p->ev[0], st));
            if ((rc = launch_chol_solve(p, 1e-7f, 1e-8f, p->scal + 1, st, p->nnp, 1, y0, r, p1, p1 ? 5e-7f : 0.0f,
                                        Dust{p->Z, r}, y1, r)))
                return rc;
            HIPCHK(hipEventRecord(p->ev[1], st));
            HIPCHK(hipEventSynchronize(p->ev[1]));
            float ms = 0.0f;
            HIPCHK(hipEventElapsedTime(&ms, p->ev[0], p->ev[1]));
            if (i > 0) total += ms;   // the first launch is untimed
        }
        *avg_ms = (float)(total / reps);
        return SPANQR_OK;
    }
    if ((rc = launch())) return rc;
    HIPCHK(hipEventRecord(p->ev[0], st));
    for (int i = 0; i < reps; ++i)
        if ((rc = launch())) return rc;
    HIPCHK(hipEventRecord(p->ev[1], st));
    HIPCHK(hipGetLastError());
    HIPCHK(hipEventSynchronize(p->ev[1]));
    float ms = 0.0f;
    HIPCHK(hipEventElapsedTime(&ms, p->ev[0], p->ev[1]));
    *avg_ms = ms / (float)reps;
    return SPANQR_OK;
}

int spanqr_stage_amax(spanqr_plan* p, const float* X, long ldx, void* stream) {
    if (!p) return fail(SPANQR_EINVAL, "plan is null");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    int rc = check_mat(p, X, ldx, "X");
    if (rc) return rc;
    DeviceGuard dg(p->device);
    launch_amax(mats_in(&X, 1), ldx, p->K, p->r, p->amax_part, nullptr, 1, (hipStream_t)stream);
    HIPCHK(hipGetLastError());
    return SPANQR_OK;
}

int spanqr_stage_gram(spanqr_plan* p, const float* A, long lda, int use_scale, int kahan, float* G, double* npart,
                      void* stream) {
    if (!p) return fail(SPANQR_EINVAL, "plan is null");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    int rc = check_mat(p, A, lda, "A");
    if (rc) return rc;
    if (!G) return fail(SPANQR_EINVAL, "G is null");
    DeviceGuard dg(p->device);
    hipStream_t st = (hipStream_t)stream;
    launch_gram_g(p, mats_in(&A, 1), lda, 1, use_scale != 0, kahan != 0, 0, st, [] { return SPANQR_OK; });
    HIPCHK(hipMemcpyAsync(G, p->G, (size_t)p->r * p->r * sizeof(float), hipMemcpyDeviceToDevice, st));
    if (npart) HIPCHK(hipMemcpyAsync(npart, p->npart, (size_t)p->nnp * sizeof(double), hipMemcpyDeviceToDevice, st));
    HIPCHK(hipGetLastError());
    return SPANQR_OK;
}

int spanqr_stage_chol(spanqr_plan* p, const float* G, const double* npart, float alpha, float tau, float* L,
                      float* Li, float* scal, void* stream) {
    if (!p || !G || !L || !Li) return fail(SPANQR_EINVAL, "null argument");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    DeviceGuard dg(p->device);
    hipStream_t st = (hipStream_t)stream;
    HIPCHK(hipMemcpyAsync(p->G, G, (size_t)p->r * p->r * sizeof(float), hipMemcpyDeviceToDevice, st));
    if (npart) HIPCHK(hipMemcpyAsync(p->npart, npart, (size_t)p->nnp * sizeof(double), hipMemcpyDeviceToDevice, st));
    k_clear_words<<<1, 64, 0, st>>>(p->bar + 2, 1, BAR_STRIDE);
    int rc = launch_chol(p, alpha, tau, p->chscal, st, npart ? p->nnp : 0, 1);
    if (rc) return rc;
    HIPCHK(hipMemcpyAsync(L, p->L, (size_t)p->r * p->r * sizeof(float), hipMemcpyDeviceToDevice, st));
    HIPCHK(hipMemcpyAsync(Li, p->Li, (size_t)p->r * CB * sizeof(float), hipMemcpyDeviceToDevice, st));
    if (scal) {
        HIPCHK(hipMemcpyAsync(scal, p->chscal, 2 * sizeof(float), hipMemcpyDeviceToDevice, st));
        HIPCHK(hipMemcpyAsync(scal + 2, p->bar + 2, sizeof(float), hipMemcpyDeviceToDevice, st));
    }
    HIPCHK(hipGetLastError());
    return SPANQR_OK;
}

int spanqr_stage_trsm(spanqr_plan* p, const float* A, long lda, int pass1, float eps, const float* L, const float* Li,
                      float* Y, long ldy, void* stream) {
    if (!p || !L || !Li) return fail(SPANQR_EINVAL, "null argument");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    int rc = check_mat(p, A, lda, "A");
    if (rc) return rc;
    if ((rc = check_mat(p, Y, ldy, "Y"))) return rc;
    DeviceGuard dg(p->device);
    hipStream_t st = (hipStream_t)stream;
    k_pack_factors<<<(int)((p->lp_stride + 255) / 256), 256, 0, st>>>(L, Li, p->r, p->Lp);
    launch_trsm(p, mats_in(&A, 1), lda, pass1 != 0, eps, Dust{p->Z, p->r}, mats_out(&Y, 1), ldy, 1, st);
    HIPCHK(hipGetLastError());
    return SPANQR_OK;
}

int spanqr_stage_ns(spanqr_plan* p, const float* Y, long ldy, int kahan, float* Yout, long ldo, void* stream) {
    if (!p) return fail(SPANQR_EINVAL, "plan is null");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    int rc = check_mat(p, Y, ldy, "Y");
    if (rc) return rc;
    if ((rc = check_mat(p, Yout, ldo, "Yout"))) return rc;
    DeviceGuard dg(p->device);
    hipStream_t st = (hipStream_t)stream;
    launch_gram_g(p, mats_in(&Y, 1), ldy, 1, false, kahan != 0, 1, st, [] { return SPANQR_OK; });
    launch_nsapply(p, mats_in(&Y, 1), ldy, mats_out(&Yout, 1), ldo, 1, st);
    HIPCHK(hipGetLastError());
    return SPANQR_OK;
}

int spanqr_profile_chol(spanqr_plan* p, const float* G, const double* npart, float alpha, float tau,
                        unsigned long long* stamps_out, double* tick_ns, void* stream) {
    if (!p || !G || !npart || !stamps_out || !tick_ns) return fail(SPANQR_EINVAL, "null argument");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    DeviceGuard dg(p->device);
    hipStream_t st = (hipStream_t)stream;
    HIPCHK(hipMemcpyAsync(p->G, G, (size_t)p->r * p->r * sizeof(float), hipMemcpyDeviceToDevice, st));
    HIPCHK(hipMemcpyAsync(p->npart, npart, (size_t)p->nnp * sizeof(double), hipMemcpyDeviceToDevice, st));
    HIPCHK(hipMemsetAsync(p->stamps, 0, (size_t)(24 * p->NB + 2) * sizeof(uint64_t), st));
    int rc = launch_chol(p, alpha, tau, p->chscal, st, p->nnp, 1, true);
    if (rc) return rc;
    HIPCHK(hipMemcpyAsync(stamps_out, p->stamps, (size_t)(24 * p->NB + 2) * sizeof(uint64_t), hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    int khz = 0;
    HIPCHK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, p->device));
    *tick_ns = khz > 0 ? 1e6 / khz : 0.0;
    return SPANQR_OK;
}

int spanqr_debug_spin_limit(unsigned polls) {
    g_spin_limit = polls;
    return SPANQR_OK;
}

int spanqr_plan_copy_dust(spanqr_plan* p, float* Z, void* stream) {
    if (!p || !Z) return fail(SPANQR_EINVAL, "null argument");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    DeviceGuard dg(p->device);
    HIPCHK(hipMemcpyAsync(Z, p->Z, (size_t)p->K * p->r * sizeof(float), hipMemcpyDeviceToDevice, (hipStream_t)stream));
    return SPANQR_OK;
}

int spanqr_plan_copy_scalars(spanqr_plan* p, float* scal8, void* stream) {
    if (!p || !scal8) return fail(SPANQR_EINVAL, "null argument");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    DeviceGuard dg(p->device);
    hipStream_t st = (hipStream_t)stream;
    HIPCHK(hipMemcpyAsync(scal8, p->scal, 7 * sizeof(float), hipMemcpyDeviceToDevice, st));
    HIPCHK(hipMemcpyAsync(scal8 + 7, p->bar + 2, sizeof(float), hipMemcpyDeviceToDevice, st));
    return SPANQR_OK;
}

int spanqr_plan_status(spanqr_plan* p, void* stream) {
    if (!p) return fail(SPANQR_EINVAL, "plan is null");
    DeviceGuard dg(p->device);
    if (!dg.ok) return fail(SPANQR_EHIP, "cannot select HIP device %d", p->device);
    const spanqr_plan* q = p->blk ? p->blk : p;
    const int n = p->blk ? 1 : (p->last_n < 1 ? 1 : p->last_n);
    const int word = p->blk ? 3 : 2;   // the column-blocked path keeps the whole call's error in word 3
    uint32_t w[SPANQR_MAX_BATCH * BAR_STRIDE];
    HIPCHK(hipMemcpyAsync(w, q->bar, (size_t)n * BAR_STRIDE * sizeof(uint32_t), hipMemcpyDeviceToHost,
                          (hipStream_t)stream));
    HIPCHK(hipStreamSynchronize((hipStream_t)stream));
    for (int i = 0; i < n; ++i)
        if (w[(size_t)i * BAR_STRIDE + word] != 0u)
            return fail(SPANQR_EHIP, "matrix %d of the last call: a bounded wait of its Cholesky gave up (not every "
                                     "workgroup of the launch was resident); its Q is NaN", i);
    return SPANQR_OK;
}

int spanqr_chol32(spanqr_plan* p, const float* G, long ldg, const float* tau, float* L, long ldl, float* Li,
                  void* stream) {
    if (!p || !G || !tau || !L || !Li) return fail(SPANQR_EINVAL, "null argument");
    if (p->blk) return fail(SPANQR_EINVAL, "not available on a column-blocked plan (r > 512)");
    const long n = p->r;
    if (ldg < n || ldl < n) return fail(SPANQR_EINVAL, "ldg = %ld, ldl = %ld: must be >= n = %ld", ldg, ldl, n);
    DeviceGuard dg(p->device);
    if (!dg.ok) return fail(SPANQR_EHIP, "cannot select HIP device %d", p->device);
    hipStream_t st = (hipStream_t)stream;
    const size_t row = (size_t)n * sizeof(float);
    HIPCHK(hipMemcpy2DAsync(p->G, row, G, (size_t)ldg * sizeof(float), row, n, hipMemcpyDeviceToDevice, st));
    k_clear_words<<<1, 64, 0, st>>>(p->bar + 2, 1, BAR_STRIDE);
    p->last_n = 1;
    int rc = launch_chol(p, 0.0f, 0.0f, nullptr, st, 0, 1, false, tau);
    if (rc) return rc;
    // L: the plan's factor, whose tiles above the diagonal no kernel writes (zero since the plan was made)
    HIPCHK(hipMemcpy2DAsync(L, (size_t)ldl * sizeof(float), p->L, row, row, n, hipMemcpyDeviceToDevice, st));
    HIPCHK(hipMemcpyAsync(Li, p->Li, (size_t)n * CB * sizeof(float), hipMemcpyDeviceToDevice, st));
    HIPCHK(hipGetLastError());
    return SPANQR_OK;
}

}  // extern "C"

// ===============================================================================================================
// Allocation-free orth: spanqr_orth_f32's kernels on a workspace carved out of a fixed device array instead of a
// plan's hipMalloc. No counterpart in the reference; for callers that cannot allocate (code under graph capture,
// serving loops). The dust is generated on the device, bit-identical to spanqr_dust_host, and kept in the array with
// a shape tag, so a call regenerates it only after a call of another shape.
// ===============================================================================================================
constexpr size_t SCRATCH_BYTES = (size_t)64 << 20;   // the largest workspace the entry point takes
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;

__device__ __forceinline__ uint64_t mix64_dev(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// raw draws of spanqr_dust_host: element e = k r + c, six splitmix64 outputs, their twelve halves summed, centred,
// scaled by 2^-32 and rounded to fp32
__global__ __launch_bounds__(256) void k_dust_raw(float* Z, int K, int r, const uint64_t* tag, uint64_t want) {
    if (*tag == want) return;
    const uint64_t key = mix64_dev(20261018ull);
    const size_t n = (size_t)K * r;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (size_t)gridDim.x * 256) {
        uint64_t S = 0;
        for (uint64_t j = 0; j < 6; ++j) {
            const uint64_t wv = mix64_dev(key + (6 * (uint64_t)e + j + 1) * 0x9E3779B97F4A7C15ull);
            S += (wv & 0xffffffffull) + (wv >> 32);
        }
        Z[e] = (float)ldexp((double)((int64_t)S - (int64_t)6 * 4294967295ll), -32);
    }
}

// column norms of the raw draws: sqrt of the squares summed in double in ascending k, one dependent chain per column.
// A workgroup takes 32 columns: its four wavefronts stream 128-row chunks of them into a ring of three LDS buffers,
// two chunks ahead, while lanes 0-31 of wave 0 run the chains over the chunk in LDS -- so the chains, not the memory
// latency of a few wavefronts' loads, set the time.
constexpr int DN_COLS = 32, DN_ROWS = 128, DN_BUF = 3;
__global__ __launch_bounds__(256) void k_dust_norm(const float* Z, int K, int r, double* nrm, const uint64_t* tag,
                                                   uint64_t want) {
    if (*tag == want) return;
    __shared__ float buf[DN_BUF][DN_ROWS][DN_COLS];
    const int c0 = blockIdx.x * DN_COLS, tid = threadIdx.x;
    const int nch = (K + DN_ROWS - 1) / DN_ROWS;
    float4 v[4];   // this thread's part of a chunk: rows (tid >> 3) + 32 u, columns 4 (tid & 7) .. + 3
    auto load = [&](int t) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int row = t * DN_ROWS + (tid >> 3) + 32 * u;
            v[u] = row < K ? *reinterpret_cast<const float4*>(Z + (size_t)row * r + c0 + 4 * (tid & 7))
                           : float4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto store = [&](int t) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            *reinterpret_cast<float4*>(&buf[t % DN_BUF][(tid >> 3) + 32 * u][4 * (tid & 7)]) = v[u];
    };
    load(0);
    store(0);
    if (nch > 1) {
        load(1);
        store(1);
    }
    __syncthreads();
    double acc = 0.0;
    for (int t = 0; t < nch; ++t) {
        if (t + 2 < nch) load(t + 2);
        if (tid < DN_COLS) {
            const int rows = K - t * DN_ROWS < DN_ROWS ? K - t * DN_ROWS : DN_ROWS;
            for (int k = 0; k < rows; ++k) {
                const double z = (double)buf[t % DN_BUF][k][tid];
                acc += z * z;
            }
        }
        // buffer (t + 2) % 3 was last read in the previous iteration, before its barrier
        if (t + 2 < nch) store(t + 2);
        __syncthreads();
    }
    if (tid < DN_COLS) nrm[c0 + tid] = sqrt(acc);
}

__global__ __launch_bounds__(256) void k_dust_scale(float* Z, int K, int r, const double* nrm, const uint64_t* tag,
                                                    uint64_t want) {
    if (*tag == want) return;
    const size_t n = (size_t)K * r;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (size_t)gridDim.x * 256)
        Z[e] = (float)((double)Z[e] / nrm[e % r]);
}

// every call: the Cholesky's flags and call counters start from zero (the previous call may have had another shape,
// hence another workgroup count), and the dust now held is tagged
__global__ __launch_bounds__(256) void k_noalloc_prep(uint32_t* flags, int nflags, uint64_t* tag, uint64_t want) {
    for (int e = threadIdx.x; e < nflags; e += 256) flags[e] = 0u;
    if (threadIdx.x == 0) *tag = want;
}

std::mutex g_na_mu;
char* g_na_base[MAX_DEVICES] = {};   // the array's device address on each device (hipGetSymbolAddress)
std::map<std::tuple<int, int, int>, spanqr_plan> g_na_setup;   // (device, K, r) -> the set-up plan fields

// The array: the dust's shape tag and column norms at fixed offsets (every call finds the tag of the dust the array
// holds at the same place, whatever the shape of the call that wrote it), then a plan's workspace.
constexpr size_t NA_TAG = 0, NA_NRM = 256, NA_WS = NA_NRM + KCH_MAX_R * sizeof(double);   // tag, dust column norms

size_t noalloc_bytes(int K, int r) {
    spanqr_plan p;
    plan_shape(&p, K, r, 1);
    return NA_WS + plan_layout(&p, nullptr);
}

}  // namespace

extern "C" {

int spanqr_orth_f32_noalloc(int K, int r, const float* X, long ldx, float* Q, long ldq, float eps, float alpha,
                            float tau, int ns, void* stream) {
    int rc = check_shape(K, r);
    if (rc != SPANQR_OK) return rc;
    if (r > 512) return fail(SPANQR_EINVAL, "noalloc: r = %d: at most 512 (use a plan)", r);
    const size_t need = noalloc_bytes(K, r);
    if (need > SCRATCH_BYTES)
        return fail(SPANQR_EINVAL, "noalloc: X [%d, %d] needs %zu bytes of workspace, more than the fixed %zu "
                                   "(use a plan)", K, r, need, SCRATCH_BYTES);
    if (ns < 0) return fail(SPANQR_EINVAL, "ns = %d < 0", ns);
    spanqr_plan p;
    plan_shape(&p, K, r, 1);
    if ((rc = check_mat(&p, X, ldx, "X"))) return rc;
    if ((rc = check_mat(&p, Q, ldq, "Q"))) return rc;
    int dev = -1;
    HIPCHK(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) return fail(SPANQR_EINVAL, "noalloc: device %d out of range", dev);
    char* base = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_na_mu);
        if (g_na_base[dev] == nullptr) {
            void* ptr = nullptr;
            HIPCHK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
            if (ptr == nullptr) return fail(SPANQR_EHIP, "noalloc: no device address for the workspace array");
            g_na_base[dev] = (char*)ptr;
        }
        base = g_na_base[dev];
    }
    p.device = dev;
    {
        // the device-derived fields of the plan (part width, co-residency, solve form), once per (device, K, r)
        std::lock_guard<std::mutex> lk(g_na_mu);
        const auto key = std::make_tuple(dev, K, r);
        const auto it = g_na_setup.find(key);
        if (it == g_na_setup.end()) {
            if ((rc = plan_device_setup(&p, dev))) return rc;
            g_na_setup.emplace(key, p);
        } else {
            p = it->second;
        }
    }
    plan_layout(&p, base + NA_WS);
    uint64_t* tag = (uint64_t*)(base + NA_TAG);
    double* nrm = (double*)(base + NA_NRM);
    const uint64_t want = ((uint64_t)(uint32_t)K << 32) | (uint32_t)r;
    hipStream_t st = (hipStream_t)stream;
    const int eblocks = (int)(((size_t)K * r + 255) / 256 < 2048 ? ((size_t)K * r + 255) / 256 : 2048);
    k_dust_raw<<<eblocks, 256, 0, st>>>(p.Z, K, r, tag, want);
    k_dust_norm<<<r / DN_COLS, 256, 0, st>>>(p.Z, K, r, nrm, tag, want);   // r is a multiple of 32
    k_dust_scale<<<eblocks, 256, 0, st>>>(p.Z, K, r, nrm, tag, want);
    k_noalloc_prep<<<1, 256, 0, st>>>(p.flags, FLAG_STRIDE, tag, want);
    HIPCHK(hipGetLastError());
    return enqueue_orth(&p, 1, mats_in(&X, 1), ldx, mats_out(&Q, 1), ldq, eps, alpha, tau, ns, st, false);
}

}  // extern "C"

// ===============================================================================================================
// fp64 clamped Cholesky (kchol.chol64, kchol.py:47-57 -> chol_f64, chol.cu:115-281 instantiated for double): the
// tile algorithm of the fp32 factorisation in double, plus fp32 copies of L and Li (chol.cu:175-176, 215, 255).
// Every workgroup owns one lower 32x32 tile (i, k) for the whole factorisation: it applies column blocks j < k in
// order, each as soon as the panels L(i, j) and L(k, j) are published (fma chains over the block's 32 columns, two
// rows x two columns per thread); then the diagonal owner factors and inverts its tile in one wavefront (the fp32
// kernel's per-column scheme in double: the pivot from lane c's register, column broadcast through LDS), and an
// off-diagonal owner forms its panel L(i, k) = T(i, k) Li_k^T (chain over the non-zero 16-column groups of Li_k)
// once Li_k is published. Publication: stores, wait for them, one agent-scope release, a flag; waits are bounded
// (an error word records a wait that gave up). Each tile waits only on tiles of earlier columns or its own column's
// diagonal tile, so with every workgroup resident (checked when the plan is made) nothing deadlocks.
// ===============================================================================================================
namespace {

constexpr int C64_TS = CB + 1;
typedef double TileD[CB][C64_TS];

__device__ __forceinline__ double readlane_d(double v, int l) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// reciprocal square root for the fp64 pivots (CUDA's rsqrt in the reference): start 0x5FE6EB50C7B537A9 - (bits >> 1)
// (the 64-bit constant published by M. Robertson, "A Brief History of InvSqrt", 2012), then four Newton steps
// y <- y * (1.5 - (0.5x * y) * y), the bracket as one fma
__device__ __forceinline__ double rsqrt64_sw(double x) {
#pragma clang fp contract(off)
    double y = __longlong_as_double((long long)(0x5FE6EB50C7B537A9ull - ((uint64_t)__double_as_longlong(x) >> 1)));
    const double h = 0.5 * x;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        double t = h * y;
        t = __builtin_fma(-t, y, 1.5);
        y = y * t;
    }
    return y;
}

// global 32x32 double tile (row stride ld) <-> LDS, all 256 threads, two doubles per access
__device__ __forceinline__ void load_tile_d(TileD& dst, const double* src, long ld) {
    for (int e = threadIdx.x; e < CB * CB / 2; e += 256) {
        const int row = e >> 4, c2 = e & 15;
        const double2 v = *reinterpret_cast<const double2*>(src + (size_t)row * ld + 2 * c2);
        dst[row][2 * c2] = v.x;
        dst[row][2 * c2 + 1] = v.y;
    }
}
// to dst (fp64) and dstf (fp32 copy), both row stride ld; lower: zeros above the diagonal
__device__ __forceinline__ void store_tile_d(double* dst, float* dstf, long ld, const TileD& src, bool lower) {
    for (int e = threadIdx.x; e < CB * CB / 2; e += 256) {
        const int row = e >> 4, c2 = e & 15;
        double2 v;
        v.x = (lower && 2 * c2 > row) ? 0.0 : src[row][2 * c2];
        v.y = (lower && 2 * c2 + 1 > row) ? 0.0 : src[row][2 * c2 + 1];
        *reinterpret_cast<double2*>(dst + (size_t)row * ld + 2 * c2) = v;
        *reinterpret_cast<float2*>(dstf + (size_t)row * ld + 2 * c2) = make_float2((float)v.x, (float)v.y);
    }
}

// T -= Pa Pb^T (chain over m = 0..31 from T); lower: elements above the diagonal are left (never read)
__device__ __forceinline__ void update_d(TileD& T, const TileD& Pa, const TileD& Pb, bool lower) {
#pragma clang fp contract(off)
    const int r0 = 2 * (threadIdx.x >> 4), c0 = 2 * (threadIdx.x & 15);
    double acc[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int v = 0; v < 2; ++v) acc[u][v] = T[r0 + u][c0 + v];
#pragma unroll 4
    for (int m = 0; m < CB; ++m) {
        const double a0 = Pa[r0][m], a1 = Pa[r0 + 1][m], b0 = Pb[c0][m], b1 = Pb[c0 + 1][m];
        acc[0][0] = __builtin_fma(-a0, b0, acc[0][0]);
        acc[0][1] = __builtin_fma(-a0, b1, acc[0][1]);
        acc[1][0] = __builtin_fma(-a1, b0, acc[1][0]);
        acc[1][1] = __builtin_fma(-a1, b1, acc[1][1]);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int v = 0; v < 2; ++v)
            if (!(lower && c0 + v > r0 + u)) T[r0 + u][c0 + v] = acc[u][v];
    __syncthreads();
}

// Out = T Li^T (chain over m < 16 (b / 16 + 1) from +0); Out may alias T
__device__ __forceinline__ void panel_d(TileD& Out, const TileD& T, const TileD& Li) {
#pragma clang fp contract(off)
    const int r0 = 2 * (threadIdx.x >> 4), c0 = 2 * (threadIdx.x & 15);
    const int mend = 16 * (c0 / 16 + 1);
    double acc[2][2] = {{0.0, 0.0}, {0.0, 0.0}};
#pragma unroll 4
    for (int m = 0; m < mend; ++m) {
        const double a0 = T[r0][m], a1 = T[r0 + 1][m], b0 = Li[c0][m], b1 = Li[c0 + 1][m];
        acc[0][0] = __builtin_fma(a0, b0, acc[0][0]);
        acc[0][1] = __builtin_fma(a0, b1, acc[0][1]);
        acc[1][0] = __builtin_fma(a1, b0, acc[1][0]);
        acc[1][1] = __builtin_fma(a1, b1, acc[1][1]);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int v = 0; v < 2; ++v) Out[r0 + u][c0 + v] = acc[u][v];
    __syncthreads();
}

// Wave 0: factor the lower part of D and invert the factor (chol.cu:131-168 in double). Lanes 0..31 hold row i of D,
// lanes 32..63 column i of the identity, which becomes column i of the inverse; column c: piv = fmax(D_cc, tau)
// (NaN -> tau) from lane c, q = rsqrt(piv), own = R[c] q (l_i on a factor lane, x_c on an inverse lane, exactly 0
// above its diagonal), then R[k] = fma(-own, l_k, R[k]) for k > c with l_k broadcast through LDS. The column loop
// is a real loop (the row stays in registers, updated under k > c), which keeps the register count low. The factor's
// diagonal entry is piv q. Writes the factor (upper triangle unspecified) to dl and the inverse to Li.
__device__ __forceinline__ void factor_inv32_d(const TileD& D, double tau, TileD& dl, TileD& Li, double* bl, double* pq) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, i = lane & 31;
    const bool fl = lane < 32;
    double R[CB];
#pragma unroll
    for (int k = 0; k < CB; ++k) R[k] = fl ? D[i][k] : (i == k ? 1.0 : 0.0);
#pragma nounroll
    for (int c = 0; c < CB; ++c) {
        double rc = 0.0;
#pragma unroll
        for (int k = 0; k < CB; ++k)
            if (k == c) rc = R[k];
        const double piv = fmax(readlane_d(rc, c), tau);
        const double q = rsqrt64_sw(piv);
        const double own = (!fl && c < i) ? 0.0 : rc * q;
        if (lane == 0) pq[c] = piv * q;
        if (fl) bl[i] = own;
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int k = 0; k < CB; ++k) {
            if (k == c) R[k] = own;
            else if (k > c) R[k] = __builtin_fma(-own, bl[k], R[k]);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int k = 0; k < CB; ++k) {
        if (fl) dl[i][k] = (k == i) ? pq[i] : R[k];
        else Li[k][i] = R[k];
    }
}

__global__ __launch_bounds__(256) void k_c64_fill(uint32_t* flags, int nf, double* L, float* Lf, int n) {
    const size_t nn = (size_t)n * n;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < nn; e += (size_t)gridDim.x * 256) {
        L[e] = 0.0;
        Lf[e] = 0.0f;
        if (e < (size_t)nf) flags[e] = 0u;
    }
}

__global__ __launch_bounds__(256) void k_chol64(const double* __restrict__ G, long ldg, int n,
                                                const double* __restrict__ taup, double* L, double* Li, float* Lf,
                                                float* Lif, uint32_t* flags) {
    extern __shared__ double c64_lds[];
    TileD* tl = reinterpret_cast<TileD*>(c64_lds);
    TileD& T = tl[0];
    TileD& Pa = tl[1];
    TileD& Pb = tl[2];
    TileD& X = tl[3];
    double* bl = c64_lds + 4 * CB * C64_TS;
    double* pq = bl + CB;
    const int u = blockIdx.x, nb = n / CB, nt = nb * (nb + 1) / 2;
    int i = 0;
    while ((i + 1) * (i + 2) / 2 <= u) ++i;
    const int k = u - i * (i + 1) / 2;
    uint32_t* err = flags + nt;
    auto fidx = [](int a, int b) { return a * (a + 1) / 2 + b; };
    bool dead = false;
    const double tau = *taup;
    load_tile_d(T, G + (size_t)CB * i * ldg + CB * k, ldg);
    __syncthreads();
    for (int j = 0; j < k; ++j) {
        if (threadIdx.x == 0) {
            wait_flag(flags + fidx(i, j), 1u, err, dead);
            if (i != k) wait_flag(flags + fidx(k, j), 1u, err, dead);
        }
        __syncthreads();
        load_tile_d(Pa, L + (size_t)CB * i * n + CB * j, n);
        if (i != k) load_tile_d(Pb, L + (size_t)CB * k * n + CB * j, n);
        __syncthreads();
        update_d(T, Pa, i == k ? Pa : Pb, i == k);
    }
    if (i == k) {
        if (threadIdx.x < 64) factor_inv32_d(T, tau, X, Pa, bl, pq);
        __syncthreads();
        store_tile_d(L + (size_t)CB * k * n + CB * k, Lf + (size_t)CB * k * n + CB * k, n, X, true);
        store_tile_d(Li + (size_t)CB * k * CB, Lif + (size_t)CB * k * CB, CB, Pa, false);
    } else {
        if (threadIdx.x == 0) wait_flag(flags + fidx(k, k), 1u, err, dead);
        __syncthreads();
        load_tile_d(Pb, Li + (size_t)CB * k * CB, CB);
        __syncthreads();
        panel_d(T, T, Pb);
        store_tile_d(L + (size_t)CB * i * n + CB * k, Lf + (size_t)CB * i * n + CB * k, n, T, false);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
    if (threadIdx.x == 0) publish_flag(flags + fidx(i, k), 1u);
}

size_t chol64_lds_bytes() { return 4 * sizeof(TileD) + 2 * CB * sizeof(double); }

}  // namespace

struct spanqr_chol64_plan {
    int n = 0, device = 0, nt = 0;
    uint32_t* flags = nullptr;   // nt tile flags + the wait-error word
};

extern "C" {

int spanqr_chol64_plan_create(int n, int device, spanqr_chol64_plan** out) {
    if (out == nullptr) return fail(SPANQR_EINVAL, "out is null");
    *out = nullptr;
    if (n < CB || n > 1024 || n % CB) return fail(SPANQR_EINVAL, "n = %d: must be a multiple of 32 in [32, 1024]", n);
    DeviceGuard dg(device);
    if (!dg.ok) return fail(SPANQR_EHIP, "cannot select HIP device %d", device);
    const int nb = n / CB, nt = nb * (nb + 1) / 2;
    int occ = 0, cus = 0;
    HIPCHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)k_chol64, 256, chol64_lds_bytes()));
    HIPCHK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
    if ((long)occ * cus < nt)
        return fail(SPANQR_EHIP, "the fp64 Cholesky needs %d resident workgroups, the device holds %d", nt, occ * cus);
    spanqr_chol64_plan* p = new spanqr_chol64_plan;
    p->n = n; p->device = device; p->nt = nt;
    if (hipMalloc((void**)&p->flags, (size_t)(nt + 1) * sizeof(uint32_t)) != hipSuccess) {
        delete p;
        return fail(SPANQR_ENOMEM, "flag allocation failed");
    }
    *out = p;
    return SPANQR_OK;
}

void spanqr_chol64_plan_destroy(spanqr_chol64_plan* p) {
    if (!p) return;
    DeviceGuard dg(p->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(p->flags);
    delete p;
}

int spanqr_chol64(spanqr_chol64_plan* p, const double* G, long ldg, const double* tau, double* L, double* Li,
                  float* Lf, float* Lif, void* stream) {
    if (!p) return fail(SPANQR_EINVAL, "plan is null");
    if (!G || !tau || !L || !Li || !Lf || !Lif) return fail(SPANQR_EINVAL, "null argument");
    if (!aligned16(G) || !aligned16(L) || !aligned16(Li) || ((uintptr_t)Lf & 7) || ((uintptr_t)Lif & 7))
        return fail(SPANQR_EINVAL, "G, L, Li must be 16-byte and Lf, Lif 8-byte aligned");
    if (ldg < p->n || (ldg & 1)) return fail(SPANQR_EINVAL, "ldg = %ld: must be >= n and even", ldg);
    DeviceGuard dg(p->device);
    if (!dg.ok) return fail(SPANQR_EHIP, "cannot select HIP device %d", p->device);
    hipStream_t st = (hipStream_t)stream;
    k_c64_fill<<<256, 256, 0, st>>>(p->flags, p->nt + 1, L, Lf, p->n);
    k_chol64<<<p->nt, 256, chol64_lds_bytes(), st>>>(G, ldg, p->n, tau, L, Li, Lf, Lif, p->flags);
    HIPCHK(hipGetLastError());
    return SPANQR_OK;
}

int spanqr_chol64_status(spanqr_chol64_plan* p, void* stream) {
    if (!p) return fail(SPANQR_EINVAL, "plan is null");
    DeviceGuard dg(p->device);
    uint32_t e = 0;
    HIPCHK(hipMemcpyAsync(&e, p->flags + p->nt, sizeof(uint32_t), hipMemcpyDeviceToHost, (hipStream_t)stream));
    HIPCHK(hipStreamSynchronize((hipStream_t)stream));
    if (e) return fail(SPANQR_EHIP, "fp64 Cholesky: a wait exceeded its bound (not every workgroup was resident)");
    return SPANQR_OK;
}

}  // extern "C"
