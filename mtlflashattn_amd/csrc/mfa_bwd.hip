// mfa_bwd.hip -- MI355X (gfx950 / CDNA4) flash-attention backward kernels and
// the mfa_bwd* entry points of include/mfa.h.
//
// The reference is forward-only (metal_flash_attn/__init__.py:3-4); these are
// the gradients of its forward semantics (metal_flash_attn/_kernel.py:32-87:
// bottom-right causal and sliding-window masks, soft-cap, ALiBi, grouped-query
// heads, varlen sequences).  With x = scale * q.k, s = cap * tanh(x / cap)
// (soft-cap) - slope * |center - j| (ALiBi), P = exp(s - lse):
//   dV = P^T dO,  dP = dO V^T,  Dsum = rowsum(dO * O),
//   dS = P * (dP - Dsum) * (1 - tanh^2)   (the last factor with soft-cap only),
//   dQ = scale * dS K,  dK = scale * dS^T Q.
//
// Three kernels, no atomics (the result does not depend on scheduling):
//  * mfa_bwd_dsum_kernel: Dsum per query row (fp32), 16 lanes per row.
//  * mfa_bwd_dkdv_kernel (head dims up to 64) / mfa_bwd_dkdv8_kernel (above):
//    a workgroup owns 128 keys of one (sequence, K/V head), 32 per
//    wavefront, with K and V resident in registers as MFMA B operands (four
//    wavefronts) or read from LDS (eight wavefronts, two per SIMD: pairs
//    that own the same keys split each step's query rows and add their
//    partial sums at the end).  It walks every query block (staged in LDS
//    with its dO, lse and Dsum) of every query head of its head group that
//    can see its keys.  S = Q K^T and dP = dO V^T come out with lane = key,
//    so P and dS feed dV^T += dO^T P and dK^T += Q^T dS straight from the
//    accumulators (rounded to 16 bits), with dO^T / Q^T read from LDS by
//    ds_read_b64_tr_b16 -- the same operand scheme as the forward's O^T.
//  * mfa_bwd_dq_kernel: a workgroup owns 128 query rows, 32 per wavefront,
//    with Q and dO resident in registers; it walks the key blocks (64 keys,
//    staged in LDS) its rows can see.  S^T = K Q^T and dP^T = V dO^T give
//    lane = query, and dQ^T += K^T dS^T takes dS^T from the accumulators.
// Tiles whose query-key pairs are all valid skip the masks; boundary tiles
// mask element-wise with selects (no branches).
// fp32 inputs run mfa_bwd32_* kernels: the same decomposition with fp32
// products on the vector ALU (see their section below).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "mfa.h"
#include "mfa_common.h"

namespace {

// 32-row query sub-blocks per dK/dV step above head dim 64.  There the
// kernel runs one wavefront per SIMD (K/V operands and dK/dV accumulators
// resident), so each step's barrier, staging and LDS latency are exposed:
// four sub-blocks (128 rows, 141 KB of LDS, no spills) amortise them over 4x
// the MFMAs (measured: fp16 B=1 L=8192 H=16 D=128 causal backward 1.43 ->
// 1.26 ms, 1.30 with two; the bf16 D=128 varlen GQA and windowed soft-cap /
// ALiBi shapes 9 % faster).
#ifndef MFA_BWD_QSB_WIDE
#define MFA_BWD_QSB_WIDE 4
#endif
// ... and at head dims up to 64 (two wavefronts per SIMD there; four:
// measured 35 % slower at bf16 B=1 L=8192 H=16 D=64)
#ifndef MFA_BWD_QSB_NARROW
#define MFA_BWD_QSB_NARROW 2
#endif
// dK/dV above head dim 64 on the eight-wavefront kernel (K/V in LDS, two
// wavefronts per SIMD) instead of the four-wavefront one
#ifndef MFA_BWD_DKDV8
#define MFA_BWD_DKDV8 1
#endif
// software-pipelined LDS operand reads in the eight-wavefront dK/dV kernel
#ifndef MFA_BWD_PREFETCH
#define MFA_BWD_PREFETCH 1
#endif
// grouped-query dK/dV: one workgroup per query head into fp32 partials
// (summed afterwards) rather than one per K/V head looping over its group
#ifndef MFA_BWD_HEAD_SPLIT
#define MFA_BWD_HEAD_SPLIT 1
#endif
// staged rows of the four-wavefront dK/dV tiles and the dQ kernel's K/V
// tiles permuted within 16-row groups (bank-conflict-free transposed reads)
#ifndef MFA_BWD_PERM
#define MFA_BWD_PERM 1
#endif
// 32-key blocks per dQ step (four: measured 17 % slower at D=128)
#ifndef MFA_BWD_DQ_NKB
#define MFA_BWD_DQ_NKB 2
#endif
constexpr int kBThreads = 256;  // 4 wavefronts

struct BArgs {
    KArgs f;  // forward arguments: q, k, v, o, strides, shapes, masks, lse (input)
    const char* dout;
    int64_t dob, dos, doh;
    char* dq;
    int64_t dqb, dqs, dqh;
    char* dk;
    int64_t dkb, dks, dkh;
    char* dv;
    int64_t dvb, dvs, dvh;
    float* dsum;       // [B*Hq][Lq] rowsum(dO * O) - dlse
    const float* dlse; // gradient of lse (softmax_lse layout), or NULL
    int32_t grad_f32;  // dq/dk/dv written as fp32
    int32_t T;         // tiles per unit (dsum: 16-row groups; dK/dV: key tiles; dQ: query tiles)
    int32_t Ukv;       // (sequence, K/V head) units = B * Hkv
    // grouped-query heads split over dK/dV workgroups: G groups of R/G query
    // heads each; G > 1 writes fp32 partials ws_dk/ws_dv [G][B*Hkv][Lk][DP]
    // that mfa_bwd_dkdv_sum_kernel adds in group order
    int32_t G;
    int32_t ws_ld;  // DP
    float* ws_dk;
    float* ws_dv;
};

// Per (sequence, query head): q, o, dO, dq, lse and Dsum rows.
struct QView {
    const char* q;
    const char* o;
    const char* dout;
    char* dq;
    const float* lse;
    float* dsum;
    int Lq, Lk;
};
__device__ __forceinline__ QView q_view(const BArgs& a, int b, int hq) {
    const KArgs& f = a.f;
    QView s;
    int64_t qs = 0, qb = 0;
    if (f.cu_q) {
        const int q0 = f.cu_q[b];
        s.Lq = f.cu_q[b + 1] - q0;
        s.Lk = f.cu_k[b + 1] - f.cu_k[b];
        qs = q0;
        s.lse = f.lse + (int64_t)hq * f.lse_h + q0;
    } else {
        s.Lq = f.Lq;
        s.Lk = f.Lk;
        qb = b;
        s.lse = f.lse + (int64_t)b * f.lse_b + (int64_t)hq * f.lse_h;
    }
    s.q = f.q + (qb * f.qb + qs * f.qs + (int64_t)hq * f.qh) * 2;
    s.o = f.o + (qb * f.ob + qs * f.os + (int64_t)hq * f.oh) * 2;
    s.dout = a.dout + (qb * a.dob + qs * a.dos + (int64_t)hq * a.doh) * 2;
    const int ges = a.grad_f32 ? 4 : 2;
    s.dq = a.dq + (qb * a.dqb + qs * a.dqs + (int64_t)hq * a.dqh) * ges;
    s.dsum = a.dsum + ((int64_t)b * f.Hq + hq) * f.Lq;
    return s;
}

// Per (sequence, K/V head): k, v, dk, dv rows.
struct KView {
    const char* k;
    const char* v;
    char* dk;
    char* dv;
    int Lk;
};
__device__ __forceinline__ KView k_view(const BArgs& a, int b, int hkv) {
    const KArgs& f = a.f;
    KView s;
    int64_t ks = 0, kb = 0;
    if (f.cu_k) {
        ks = f.cu_k[b];
        s.Lk = f.cu_k[b + 1] - f.cu_k[b];
    } else {
        kb = b;
        s.Lk = f.Lk;
    }
    s.k = f.k + (kb * f.kb + ks * f.ks + (int64_t)hkv * f.kh) * 2;
    s.v = f.v + (kb * f.vb + ks * f.vs + (int64_t)hkv * f.vh) * 2;
    const int ges = a.grad_f32 ? 4 : 2;
    s.dk = a.dk + (kb * a.dkb + ks * a.dks + (int64_t)hkv * a.dkh) * ges;
    s.dv = a.dv + (kb * a.dvb + ks * a.dvs + (int64_t)hkv * a.dvh) * ges;
    return s;
}

// Row permutation within 16-row groups for padded tiles of row stride
// D + 8 elements (D/8 + 1 16-byte chunks, = 1 mod 4): row r is stored at
// LDS row prow(r) = 4*(r mod 4) + (r/4) mod 4 of its group.  The 16 rows a
// row read covers per pass then start in 16 distinct 4-bank groups (any odd
// stride permutes the residues), and the 4 rows x 4 chunks of a transposed
// read's pass fall on 4*(r mod 4) + chunk + const: 16 distinct groups too.
__device__ __forceinline__ int prow(int r) { return (r & ~15) | ((r & 3) << 2) | ((r >> 2) & 3); }

template <bool IS_BF16>
struct Ops {
    typedef typename std::conditional<IS_BF16, bf16x8_t, f16x8_t>::type op_t;
    __device__ static __forceinline__ f32x16_t mfma(const op_t& x, const op_t& y, const f32x16_t& acc) {
        if constexpr (IS_BF16)
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, acc, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(x, y, acc, 0, 0, 0);
    }
    // two floats rounded to 16 bits, packed
    __device__ static __forceinline__ uint32_t pack(float x, float y) {
        if constexpr (IS_BF16) {
            typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 v2;
            const v2 p = {(__bf16)x, (__bf16)y};
            return __builtin_bit_cast(uint32_t, p);
        } else {
            typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 v2;
            const v2 p = {(_Float16)x, (_Float16)y};
            return __builtin_bit_cast(uint32_t, p);
        }
    }
    __device__ static __forceinline__ float to_f(uint16_t h) {
        if constexpr (IS_BF16)
            return __uint_as_float((uint32_t)h << 16);
        else
            return (float)__builtin_bit_cast(_Float16, h);
    }
    // A/B operand of the 32x32x16 MFMA whose lanes hold rows r0..r0+3 and
    // r0+8..r0+11 (this lane's k-slots) of column `col` of a row-major LDS
    // tile with row stride `st` elements (two ds_read_b64_tr_b16: in each
    // 16-lane group lane i addresses 4 elements of row i/4 and receives
    // element i%16 of rows 0..3).
    __device__ static __forceinline__ op_t load_tr(const uint16_t* tile, int st, int r0, int c0, int lane) {
        const int tr_row = 4 * (lane >> 5) + ((lane & 15) >> 2);
        const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
        const uint16_t* p0 = tile + (r0 + tr_row) * st + c0 + tr_col;
        return load_tr_rows(p0, p0 + 8 * st);
    }
    // load_tr on a tile whose rows are stored permuted within 16-row groups
    // (row r at LDS row prow(r)); r0 is a multiple of 16
    __device__ static __forceinline__ op_t load_tr_perm(const uint16_t* tile, int st, int r0, int c0, int lane) {
        const int tr_row = 4 * (lane >> 5) + ((lane & 15) >> 2);
        const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
        const uint16_t* base = tile + r0 * st + c0 + tr_col;
        return load_tr_rows(base + prow(tr_row) * st, base + prow(tr_row + 8) * st);
    }
    // the same from this lane's two addresses (row tr_row and tr_row + 8)
    __device__ static __forceinline__ op_t load_tr_rows(const uint16_t* p0, const uint16_t* p1) {
        if constexpr (IS_BF16) {
            typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 v4;
            typedef __attribute__((address_space(3))) v4* lp;
            const v4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lp)(p0));
            const v4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lp)(p1));
            return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        } else {
            typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 v4h;
            typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 v4;
            typedef __attribute__((address_space(3))) v4h* lp;
            const v4 lo = __builtin_bit_cast(v4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lp)(p0)));
            const v4 hi = __builtin_bit_cast(v4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lp)(p1)));
            return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    }
};

// Soft-cap and ALiBi of one raw score (natural-log units), and the soft-cap
// derivative factor 1 - tanh^2 (1 without soft-cap).
template <bool BIAS>
__device__ __forceinline__ float transform(const KArgs& f, float x, float slope, float dist, float& dcap) {
    dcap = 1.f;
    if constexpr (BIAS) {
        // one multiply: by the scale, or under soft-cap straight by the
        // exponent's constant (the scale folded in, as in the forward):
        // tanh(scale*x / cap) = 1 - 2 / (exp2(x * softcap_sk) + 1)
        const bool cap = f.softcap > 0.f;
        x *= cap ? f.softcap_sk : f.scale;
        if (cap) {
            const float t = 1.f - 2.f * __builtin_amdgcn_rcpf(fast_exp2(x) + 1.f);
            x = f.softcap * t;
            dcap = 1.f - t * t;
        }
        if (f.alibi) x = fmaf(-slope, fabsf(dist), x);
    }
    return x;
}

// exp2-domain lse of a row for P = exp2(s*c - lse2): lse*log2(e), and +inf for
// a row with no valid key (so its P is 0).
__device__ __forceinline__ float lse2_of(float lse) { return lse == -INFINITY ? INFINITY : lse * kLog2e; }

// ----------------------------------------------------------------------------
// Dsum = rowsum(dO * O) in fp32: 16 lanes per row, 8 elements per lane.
template <bool IS_BF16>
__global__ void __launch_bounds__(kBThreads) mfa_bwd_dsum_kernel(BArgs a) {
    const int bid = blockIdx.x;
    const int unit = bid / a.T, tile = bid - unit * a.T;
    const int b = unit / a.f.Hq, hq = unit - b * a.f.Hq;
    const QView qv = q_view(a, b, hq);
    const int row = tile * 16 + (threadIdx.x >> 4), sub = threadIdx.x & 15;
    float acc = 0.f;
    const int d0 = sub * 8;
    if (row < qv.Lq && d0 < a.f.D) {
        const u32x4_t o = *reinterpret_cast<const u32x4_t*>(qv.o + ((int64_t)row * a.f.os + d0) * 2);
        const u32x4_t g = *reinterpret_cast<const u32x4_t*>(qv.dout + ((int64_t)row * a.dos + d0) * 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc = fmaf(Ops<IS_BF16>::to_f((uint16_t)(o[i] & 0xffff)), Ops<IS_BF16>::to_f((uint16_t)(g[i] & 0xffff)), acc);
            acc = fmaf(Ops<IS_BF16>::to_f((uint16_t)(o[i] >> 16)), Ops<IS_BF16>::to_f((uint16_t)(g[i] >> 16)), acc);
        }
    }
    acc += __shfl_xor(acc, 8);
    acc += __shfl_xor(acc, 4);
    acc += __shfl_xor(acc, 2);
    acc += __shfl_xor(acc, 1);
    if (sub == 0 && row < qv.Lq) {
        if (a.dlse) {  // d lse / d s = P: enters as Dsum - dlse (same offset as the lse row)
            const float* dl = a.dlse + (qv.lse - a.f.lse);
            acc -= dl[row];
        }
        qv.dsum[row] = acc;
    }
}

// Store rows of a transposed accumulator (lane = row `idx` of the output,
// registers = columns d = 32*db + 8*g + 4*half + 0..3), scaled.
template <int DB>
__device__ __forceinline__ void store_rows(char* base, int64_t row_stride, int D, bool f32out, bool is_bf16,
                                           const f32x16_t (&acc)[DB], float scale, int half) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * db + 8 * g + 4 * half;
            if (d >= D) continue;
            const float v0 = acc[db][4 * g] * scale, v1 = acc[db][4 * g + 1] * scale;
            const float v2 = acc[db][4 * g + 2] * scale, v3 = acc[db][4 * g + 3] * scale;
            if (f32out) {
                *reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + d) = make_float4(v0, v1, v2, v3);
            } else if (is_bf16) {
                typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 v4;
                const v4 w = {(__bf16)v0, (__bf16)v1, (__bf16)v2, (__bf16)v3};
                *reinterpret_cast<v4*>(reinterpret_cast<__bf16*>(base) + d) = w;
            } else {
                typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 v4;
                const v4 w = {(_Float16)v0, (_Float16)v1, (_Float16)v2, (_Float16)v3};
                *reinterpret_cast<v4*>(reinterpret_cast<_Float16*>(base) + d) = w;
            }
        }
    (void)row_stride;
}

// ----------------------------------------------------------------------------
// dK / dV: workgroup = 128 keys of one (sequence, K/V head), 32 per wavefront.
template <int DP, bool IS_BF16, bool BIAS>
__global__ void __launch_bounds__(kBThreads) __attribute__((amdgpu_waves_per_eu(1)))
mfa_bwd_dkdv_kernel(BArgs a) {
    typedef Ops<IS_BF16> O;
    typedef typename O::op_t op_t;
    constexpr int DS = DP / 16, DB = DP / 32;
    // query rows per step: QSB 32-row sub-blocks (the per-step barrier,
    // staging and lse/Dsum loads serve QSB times the MFMAs): two at head
    // dims up to 64, where the registers allow two wavefronts per SIMD with
    // them, MFA_BWD_QSB_WIDE above
    constexpr int QSB = DP <= 64 ? MFA_BWD_QSB_NARROW : MFA_BWD_QSB_WIDE;
    // At DP <= 64 (two wavefronts per SIMD, which hide the extra LDS read
    // before the first MFMA) Dsum is staged negated and dP starts from it, so
    // the accumulator ends as dP - Dsum; at larger DP Dsum is subtracted from
    // the finished dP.
    constexpr bool DFOLD = DP <= 64;
    constexpr int BQ = 32 * QSB;
    static_assert(BQ <= 128, "the host bounds a staged block's byte span for 128 rows");
    constexpr int QST = DP + 8;  // LDS row stride of the Q / dO tiles (elements)
    constexpr int CPR = DP / 8;  // 16-byte chunks per row
    constexpr int SCH = (BQ * CPR + kBThreads - 1) / kBThreads;  // staged chunks per thread and tensor
    // two stages: the next query block is loaded while this one is computed
    __shared__ __attribute__((aligned(16))) uint16_t q_s[2][BQ * QST];
    __shared__ __attribute__((aligned(16))) uint16_t do_s[2][BQ * QST];
    __shared__ __attribute__((aligned(16))) float lse_s[2][BQ];
    __shared__ __attribute__((aligned(16))) float ds_s[2][BQ];

    const KArgs& f = a.f;
    const int bid = blockIdx.x;
    const int ktile = bid / (a.Ukv * a.G), rem = bid - ktile * (a.Ukv * a.G);
    const int unit = rem / a.G, grp = rem - unit * a.G;
    const int b = unit / f.Hkv, hkv = unit - b * f.Hkv;
    const KView kv = k_view(a, b, hkv);
    const int Lk = kv.Lk, D = f.D;
    const int k0 = ktile * 128;
    if (k0 >= Lk) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int key = k0 + wave * 32 + l32;  // this lane's key (B-operand / accumulator column)
    const int k1 = min(k0 + 128, Lk) - 1;

    // K and V rows of this lane's key as B operands (k-slots d = 16*s + 8*half + 0..7)
    op_t kf[DS], vf[DS];
#pragma unroll
    for (int s = 0; s < DS; ++s) {
        const int d = 16 * s + 8 * half;
        u32x4_t kk = {0, 0, 0, 0}, vv = {0, 0, 0, 0};
        if (key < Lk && d < D) {
            kk = *reinterpret_cast<const u32x4_t*>(kv.k + ((int64_t)key * f.ks + d) * 2);
            vv = *reinterpret_cast<const u32x4_t*>(kv.v + ((int64_t)key * f.vs + d) * 2);
        }
        kf[s] = __builtin_bit_cast(op_t, kk);
        vf[s] = __builtin_bit_cast(op_t, vv);
    }
    f32x16_t dka[DB], dva[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dka[db][r] = dva[db][r] = 0.f;
    const float c = BIAS ? kLog2e : f.scale_log2;

    // Query blocks: every head of the K/V group, the blocks whose rows can
    // see [k0, k1] (the same range for every head: lengths are per sequence).
    const int R = f.Hq / f.Hkv / a.G;       // query heads of this workgroup
    const int hq0 = hkv * R * a.G + grp * R;  // the first of them
    const int Lq = f.cu_q ? f.cu_q[b + 1] - f.cu_q[b] : f.Lq;
    const int dq = Lk - Lq;
    int qlo = 0, qhi = Lq - 1;
    if (f.causal) qlo = max(qlo, k0 - dq);
    if (f.wr >= 0) qlo = max(qlo, k0 - f.wr - dq);
    if (f.wl >= 0) qhi = min(qhi, k1 + f.wl - dq);
    const int qb0 = (qlo / BQ) * BQ;
    const int nqb = qhi >= qb0 ? (qhi - qb0) / BQ + 1 : 0;
    const int nsteps = R * nqb;

    // Staging through buffer loads: one resource per tensor and block, sized
    // to the block's valid rows (rows past the sequence and chunks past the
    // head dim read zero), so the loads carry no per-chunk conditions.
    u32x4_t sq[SCH], sd[SCH];
    uint32_t qoff[SCH], dooff[SCH];
    int soff[SCH];
#pragma unroll
    for (int i = 0; i < SCH; ++i) {
        const int cc = tid + kBThreads * i;
        const int row = cc / CPR, col = (cc % CPR) * 8;
        const bool in = cc < BQ * CPR && col < D;
        qoff[i] = in ? (uint32_t)(((int64_t)row * f.qs + col) * 2) : 0x80000000u;
        dooff[i] = in ? (uint32_t)(((int64_t)row * a.dos + col) * 2) : 0x80000000u;
        soff[i] = (MFA_BWD_PERM ? prow(row) : row) * QST + col;
    }
    float lreg = INFINITY, dreg = 0.f;
    // step order: query head rr (of the R), then its query blocks qi; the
    // load runs one step ahead of the compute, each with a cursor of its own
    // (no per-step division)
    int l_rr = 0, l_qi = 0;
    auto gload = [&]() {
        const int q0 = qb0 + l_qi * BQ;
        const QView qv = q_view(a, b, hq0 + l_rr);
        if (++l_qi == nqb) {
            l_qi = 0;
            ++l_rr;
        }
        const int rm1 = min(Lq - q0, BQ) - 1;  // q0 < Lq
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(qv.q + (int64_t)q0 * f.qs * 2), (short)0, (int)(((int64_t)rm1 * f.qs + D) * 2), kBufferDword3);
        const __amdgpu_buffer_rsrc_t dr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(qv.dout + (int64_t)q0 * a.dos * 2), (short)0, (int)(((int64_t)rm1 * a.dos + D) * 2), kBufferDword3);
#pragma unroll
        for (int i = 0; i < SCH; ++i) {
            sq[i] = __builtin_amdgcn_raw_buffer_load_b128(qr, qoff[i], 0, 0);
            sd[i] = __builtin_amdgcn_raw_buffer_load_b128(dr, dooff[i], 0, 0);
        }
        if (tid < BQ) {
            const bool in = q0 + tid < Lq;
            lreg = in ? lse2_of(qv.lse[q0 + tid]) : INFINITY;
            const float dsv = in ? qv.dsum[q0 + tid] : 0.f;
            dreg = DFOLD ? -dsv : dsv;
        }
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int i = 0; i < SCH; ++i) {
            if (SCH * kBThreads == BQ * CPR || tid + kBThreads * i < BQ * CPR) {
                *reinterpret_cast<u32x4_t*>(q_s[buf] + soff[i]) = sq[i];
                *reinterpret_cast<u32x4_t*>(do_s[buf] + soff[i]) = sd[i];
            }
        }
        if (tid < BQ) {
            lse_s[buf][tid] = lreg;
            ds_s[buf][tid] = dreg;
        }
    };
    if (nsteps > 0) {
        gload();
        swrite(0);
    }
    __syncthreads();
    int rr = 0, qi = 0;  // the step computed
    for (int step = 0; step < nsteps; ++step) {
        const int buf = step & 1;
        if (step + 1 < nsteps) gload();  // in flight during this step's MFMAs
        const int q0 = qb0 + qi * BQ;
        const int hq = hq0 + rr;
        if (++qi == nqb) {
            qi = 0;
            ++rr;
        }
        const float slope = BIAS && f.alibi ? f.alibi[b * f.alibi_bstride + hq] : 0.f;
        {
            const uint16_t* qsb = q_s[buf];
            const uint16_t* dosb = do_s[buf];

            // S = Q K^T and dP = dO V^T per 32-row sub-block (lane = key,
            // registers = query rows)
            f32x16_t sacc[QSB], dpacc[QSB];
#pragma unroll
            for (int sb = 0; sb < QSB; ++sb)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 d4 = DFOLD ? *reinterpret_cast<const float4*>(ds_s[buf] + 32 * sb + 8 * g + 4 * half)
                                            : float4{0.f, 0.f, 0.f, 0.f};
                    dpacc[sb][4 * g] = d4.x;
                    dpacc[sb][4 * g + 1] = d4.y;
                    dpacc[sb][4 * g + 2] = d4.z;
                    dpacc[sb][4 * g + 3] = d4.w;
#pragma unroll
                    for (int i = 0; i < 4; ++i) sacc[sb][4 * g + i] = 0.f;
                }
#pragma unroll
            for (int s = 0; s < DS; ++s)
#pragma unroll
                for (int sb = 0; sb < QSB; ++sb) {
                    const int row = 32 * sb + l32;
                    const int prw = MFA_BWD_PERM ? prow(row) : row;
                    const op_t qa = *reinterpret_cast<const op_t*>(qsb + prw * QST + 16 * s + 8 * half);
                    const op_t da = *reinterpret_cast<const op_t*>(dosb + prw * QST + 16 * s + 8 * half);
                    sacc[sb] = O::mfma(qa, kf[s], sacc[sb]);
                    dpacc[sb] = O::mfma(da, vf[s], dpacc[sb]);
                }
            // Per sub-block: P and dS, rounded to 16 bits for the MFMAs (register
            // r is query q0 + 32*sb + acc_row(r) + 4*half; tiles whose 32 x 32
            // pairs are all valid, a wave-uniform test since lo/hi grow with
            // the query, skip the masks), then the dV / dK products.
            const int wk0 = k0 + wave * 32;
            // (a compile-time loop: a run-time one, even unrolled, costs SGPR
            // spills inside the step loop)
            static_for<QSB>([&](auto sbc) __attribute__((always_inline)) {
                constexpr int sb = decltype(sbc)::value;
                uint32_t pw[8], dw[8];
                const int qs0 = q0 + 32 * sb;
                const bool full = qs0 + 32 <= Lq && key_lo(f, qs0 + 31 + dq) <= wk0 && key_hi(f, qs0 + dq, Lk) >= wk0 + 31;
                auto probs = [&](auto masked_tag) {
                    constexpr bool MASKED = decltype(masked_tag)::value;
                    // ALiBi distance center - key of register r: this lane's
                    // base plus the register's row offset, exact in fp32
                    // below 2^24 (formed in each path: the pin keeps the
                    // per-register values from being hoisted above the branch)
                    float dist0 = (float)(qs0 + 4 * half + dq - key);
                    asm volatile("" : "+v"(dist0));
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const float4 l4 = *reinterpret_cast<const float4*>(lse_s[buf] + 32 * sb + 8 * g + 4 * half);
                        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
                        const float4 d4 = DFOLD ? float4{0.f, 0.f, 0.f, 0.f}
                                                : *reinterpret_cast<const float4*>(ds_s[buf] + 32 * sb + 8 * g + 4 * half);
                        const float dv4[4] = {d4.x, d4.y, d4.z, d4.w};
                        float p[4], ds[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int r = 4 * g + i;
                            const int q = qs0 + acc_row(r) + 4 * half;
                            const int center = q + dq;
                            float dcap;
                            const float x = transform<BIAS>(f, sacc[sb][r], slope, dist0 + (float)acc_row(r), dcap);
                            // (bitwise tests and an unconditional exp: selects, no branches)
                            const float pe = fast_exp2(fmaf(x, c, -lv[i]));
                            bool ok = true;
                            if constexpr (MASKED)
                                ok = (key <= key_hi(f, center, Lk)) & (key >= key_lo(f, center)) & (q < Lq);
                            p[i] = ok ? pe : 0.f;
                            ds[i] = DFOLD ? p[i] * dpacc[sb][r] : p[i] * (dpacc[sb][r] - dv4[i]);
                            if constexpr (BIAS) ds[i] *= dcap;
                        }
                        pw[2 * g] = O::pack(p[0], p[1]);
                        pw[2 * g + 1] = O::pack(p[2], p[3]);
                        dw[2 * g] = O::pack(ds[0], ds[1]);
                        dw[2 * g + 1] = O::pack(ds[2], ds[3]);
                    }
                };
                if (full)
                    probs(std::false_type{});
                else
                    probs(std::true_type{});
                // dV^T += dO^T P, dK^T += Q^T dS: k-slots = query rows of accumulator
                // registers 8*st..8*st+7 (rows 32*sb + 16*st + 4*half + 0..3, +8..11)
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const u32x4_t pv = {pw[4 * st], pw[4 * st + 1], pw[4 * st + 2], pw[4 * st + 3]};
                    const u32x4_t dsv = {dw[4 * st], dw[4 * st + 1], dw[4 * st + 2], dw[4 * st + 3]};
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        const op_t dot = MFA_BWD_PERM ? O::load_tr_perm(dosb, QST, 32 * sb + 16 * st, 32 * db, lane)
                                                      : O::load_tr(dosb, QST, 32 * sb + 16 * st, 32 * db, lane);
                        const op_t qt = MFA_BWD_PERM ? O::load_tr_perm(qsb, QST, 32 * sb + 16 * st, 32 * db, lane)
                                                     : O::load_tr(qsb, QST, 32 * sb + 16 * st, 32 * db, lane);
                        dva[db] = O::mfma(dot, __builtin_bit_cast(op_t, pv), dva[db]);
                        dka[db] = O::mfma(qt, __builtin_bit_cast(op_t, dsv), dka[db]);
                    }
                }
            });
        }
        if (step + 1 < nsteps) swrite(buf ^ 1);  // the other stage was last read before the previous barrier
        __syncthreads();
    }
    if (key < Lk) {
        if (a.G > 1) {  // this group's partial sums, unscaled, fp32
            const int64_t row = ((int64_t)grp * a.Ukv + unit) * f.Lk + key;
            store_rows<DB>(reinterpret_cast<char*>(a.ws_dk + row * a.ws_ld), 0, D, true, IS_BF16, dka, 1.f, half);
            store_rows<DB>(reinterpret_cast<char*>(a.ws_dv + row * a.ws_ld), 0, D, true, IS_BF16, dva, 1.f, half);
        } else {
            const bool f32o = a.grad_f32 != 0;
            const int ges = f32o ? 4 : 2;
            store_rows<DB>(kv.dk + (int64_t)key * a.dks * ges, 0, D, f32o, IS_BF16, dka, f.scale, half);
            store_rows<DB>(kv.dv + (int64_t)key * a.dvs * ges, 0, D, f32o, IS_BF16, dva, 1.f, half);
        }
    }
}

// ----------------------------------------------------------------------------
// dK / dV above head dim 64 on eight wavefronts (two per SIMD): workgroup =
// 128 keys of one (sequence, K/V head).  Wavefronts w and w+4 own the same 32
// keys and take the two 32-row sub-blocks of each 64-row query step, so each
// wavefront computes S, dP, dV and dK for one sub-block per step.  K and V
// sit in LDS (read as MFMA B operands like the Q / dO rows), which leaves
// room for two wavefronts per SIMD: while one waits on a barrier, staging or
// an LDS read, the other's MFMAs run.  Each wavefront of the pair holds a
// partial dK / dV over its sub-blocks; the pair's sums are added in a fixed
// order (w + (w+4)) through LDS at the end, so the result does not depend
// on scheduling.  dP starts from -Dsum (staged negated), so dS = P * dP.
constexpr int kB8Threads = 512;  // 8 wavefronts
template <int DP, bool IS_BF16, bool BIAS>
__global__ void __launch_bounds__(kB8Threads) mfa_bwd_dkdv8_kernel(BArgs a) {
    typedef Ops<IS_BF16> O;
    typedef typename O::op_t op_t;
    constexpr int DS = DP / 16, DB = DP / 32;
    constexpr int NT = kB8Threads;
    constexpr int BQ = 64;       // query rows per step (two sub-blocks)
    constexpr int ST = DP + 8;   // LDS row stride (elements) of the K / V tiles
    constexpr int CPR = DP / 8;  // 16-byte chunks per row
    // Staged Q / dO rows start at chunk 20*row + (row/4)%4 (16-byte chunks):
    // the start's residue mod 16 chunks (the 64 banks) is 4*(row%4) +
    // (row/4)%4, distinct over 16 consecutive rows, so the row reads (16 rows,
    // one chunk each per 256-byte pass) and the transposed reads (4 rows x 4
    // chunks per pass) both hit 16 distinct 4-bank groups; rows 16 apart
    // differ by a constant 2560 elements and rows 8 apart (within 4-row
    // groups 0/1 of each 16) by 1296.
    constexpr int QT = (20 * BQ + 4) * 8;  // elements per staged Q / dO tile
    auto rstart = [](int row) { return (20 * row + ((row >> 2) & 3)) * 8; };
    constexpr int SCH = (BQ * CPR + NT - 1) / NT;   // staged chunks per thread and tensor
    constexpr int KCH = (128 * CPR + NT - 1) / NT;  // K (and V) chunks per thread
    // K rows [0, 128) then V rows; reused for the pair sums at the end
    __shared__ __attribute__((aligned(16))) uint16_t kv_s[2 * 128 * ST];
    static_assert(sizeof(kv_s) >= 4 * DB * 16 * 64 * sizeof(float), "pair-sum buffer");
    __shared__ __attribute__((aligned(16))) uint16_t q_s[2][QT];
    __shared__ __attribute__((aligned(16))) uint16_t do_s[2][QT];
    __shared__ __attribute__((aligned(16))) float lse_s[2][BQ];
    __shared__ __attribute__((aligned(16))) float ds_s[2][BQ];

    const KArgs& f = a.f;
    const int bid = blockIdx.x;
    const int ktile = bid / (a.Ukv * a.G), rem = bid - ktile * (a.Ukv * a.G);
    const int unit = rem / a.G, grp = rem - unit * a.G;
    const int b = unit / f.Hkv, hkv = unit - b * f.Hkv;
    const KView kv = k_view(a, b, hkv);
    const int Lk = kv.Lk, D = f.D;
    const int k0 = ktile * 128;
    if (k0 >= Lk) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kw = wave & 3, sb = wave >> 2;  // key block, query sub-block of each step
    const int l32 = lane & 31, half = lane >> 5;
    const int key = k0 + kw * 32 + l32;  // this lane's key (B-operand / accumulator column)
    const int k1 = min(k0 + 128, Lk) - 1;

    // K and V rows of the workgroup into LDS (rows past the sequence and
    // columns past the head dim as zeros); every chunk of this thread is
    // loaded before any is stored, one memory round trip for all of them
    {
        u32x4_t kk[KCH], vv[KCH];
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int cc = tid + NT * i;
            const int row = cc / CPR, col = (cc % CPR) * 8;
            kk[i] = vv[i] = u32x4_t{0, 0, 0, 0};
            if (cc < 128 * CPR && k0 + row < Lk && col < D) {
                kk[i] = *reinterpret_cast<const u32x4_t*>(kv.k + ((int64_t)(k0 + row) * f.ks + col) * 2);
                vv[i] = *reinterpret_cast<const u32x4_t*>(kv.v + ((int64_t)(k0 + row) * f.vs + col) * 2);
            }
        }
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int cc = tid + NT * i;
            if (KCH * NT == 128 * CPR || cc < 128 * CPR) {
                const int row = cc / CPR, col = (cc % CPR) * 8;
                *reinterpret_cast<u32x4_t*>(kv_s + row * ST + col) = kk[i];
                *reinterpret_cast<u32x4_t*>(kv_s + (128 + row) * ST + col) = vv[i];
            }
        }
    }
    f32x16_t dka[DB], dva[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dka[db][r] = dva[db][r] = 0.f;
    const float c = BIAS ? kLog2e : f.scale_log2;

    // query blocks: as in mfa_bwd_dkdv_kernel, in 64-row steps
    const int R = f.Hq / f.Hkv / a.G;
    const int hq0 = hkv * R * a.G + grp * R;
    const int Lq = f.cu_q ? f.cu_q[b + 1] - f.cu_q[b] : f.Lq;
    const int dq = Lk - Lq;
    int qlo = 0, qhi = Lq - 1;
    if (f.causal) qlo = max(qlo, k0 - dq);
    if (f.wr >= 0) qlo = max(qlo, k0 - f.wr - dq);
    if (f.wl >= 0) qhi = min(qhi, k1 + f.wl - dq);
    const int qb0 = (qlo / BQ) * BQ;
    const int nqb = qhi >= qb0 ? (qhi - qb0) / BQ + 1 : 0;
    const int nsteps = R * nqb;

    // buffer-load staging of Q / dO (rows past the sequence read zero)
    u32x4_t sq[SCH], sd[SCH];
    uint32_t qoff[SCH], dooff[SCH];
    int soff[SCH];
#pragma unroll
    for (int i = 0; i < SCH; ++i) {
        const int cc = tid + NT * i;
        const int row = cc / CPR, col = (cc % CPR) * 8;
        const bool in = cc < BQ * CPR && col < D;
        qoff[i] = in ? (uint32_t)(((int64_t)row * f.qs + col) * 2) : 0x80000000u;
        dooff[i] = in ? (uint32_t)(((int64_t)row * a.dos + col) * 2) : 0x80000000u;
        soff[i] = rstart(row) + col;
    }
    float lreg = INFINITY, dreg = 0.f;
    // step order: query head rr (of the R), then its query blocks qi; the
    // load runs one step ahead of the compute, each with a cursor of its own
    // (no per-step division)
    int l_rr = 0, l_qi = 0;
    auto gload = [&]() {
        const int q0 = qb0 + l_qi * BQ;
        const QView qv = q_view(a, b, hq0 + l_rr);
        if (++l_qi == nqb) {
            l_qi = 0;
            ++l_rr;
        }
        const int rm1 = min(Lq - q0, BQ) - 1;  // q0 < Lq
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(qv.q + (int64_t)q0 * f.qs * 2), (short)0, (int)(((int64_t)rm1 * f.qs + D) * 2), kBufferDword3);
        const __amdgpu_buffer_rsrc_t dr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(qv.dout + (int64_t)q0 * a.dos * 2), (short)0, (int)(((int64_t)rm1 * a.dos + D) * 2), kBufferDword3);
#pragma unroll
        for (int i = 0; i < SCH; ++i) {
            sq[i] = __builtin_amdgcn_raw_buffer_load_b128(qr, qoff[i], 0, 0);
            sd[i] = __builtin_amdgcn_raw_buffer_load_b128(dr, dooff[i], 0, 0);
        }
        if (tid < BQ) {
            const bool in = q0 + tid < Lq;
            lreg = in ? lse2_of(qv.lse[q0 + tid]) : INFINITY;
            dreg = in ? -qv.dsum[q0 + tid] : 0.f;
        }
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int i = 0; i < SCH; ++i) {
            if (SCH * NT == BQ * CPR || tid + NT * i < BQ * CPR) {
                *reinterpret_cast<u32x4_t*>(q_s[buf] + soff[i]) = sq[i];
                *reinterpret_cast<u32x4_t*>(do_s[buf] + soff[i]) = sd[i];
            }
        }
        if (tid < BQ) {
            lse_s[buf][tid] = lreg;
            ds_s[buf][tid] = dreg;
        }
    };
    if (nsteps > 0) {
        gload();
        swrite(0);
    }
    __syncthreads();
    const uint16_t* kbase = kv_s + (32 * kw + l32) * ST + 8 * half;  // this lane's K row
    const uint16_t* vbase = kbase + 128 * ST;                         // and V row
    const int wk0 = k0 + kw * 32;
    // this lane's staged-row offsets: row 32*sb + l32 (A operands of S, dP)
    // and, for the transposed reads, row 32*sb + tr_row, column tr_col
    const int rq = rstart(32 * sb + l32) + 8 * half;
    const int tr_row = 4 * half + ((lane & 15) >> 2);
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int rt = rstart(32 * sb + tr_row) + tr_col;
    int rr = 0, qi = 0;  // the step computed
    for (int step = 0; step < nsteps; ++step) {
        const int buf = step & 1;
        if (step + 1 < nsteps) gload();  // in flight during this step's MFMAs
        const int qs0 = qb0 + qi * BQ + 32 * sb;  // this wavefront's first query row
        const int hq = hq0 + rr;
        if (++qi == nqb) {
            qi = 0;
            ++rr;
        }
        const float slope = BIAS && f.alibi ? f.alibi[b * f.alibi_bstride + hq] : 0.f;
        const uint16_t* qsb = q_s[buf];
        const uint16_t* dosb = do_s[buf];
        const float* lsb = lse_s[buf] + 32 * sb;
        const float* dsb = ds_s[buf] + 32 * sb;

        // S = Q K^T and dP = dO V^T - Dsum (lane = key, registers = query rows)
        f32x16_t sacc, dpacc;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 d4 = *reinterpret_cast<const float4*>(dsb + 8 * g + 4 * half);
            dpacc[4 * g] = d4.x;
            dpacc[4 * g + 1] = d4.y;
            dpacc[4 * g + 2] = d4.z;
            dpacc[4 * g + 3] = d4.w;
#pragma unroll
            for (int i = 0; i < 4; ++i) sacc[4 * g + i] = 0.f;
        }
        // operand fragments are read one MFMA pair ahead (the sched_barriers
        // keep the compiler from sinking each read to just before its MFMA,
        // which exposed the LDS latency at every pair)
        op_t fq[2], fk[2], fd[2], fv[2];
        auto ld_sdp = [&](int s, int i) __attribute__((always_inline)) {
            fq[i] = *reinterpret_cast<const op_t*>(qsb + rq + 16 * s);
            fk[i] = *reinterpret_cast<const op_t*>(kbase + 16 * s);
            fd[i] = *reinterpret_cast<const op_t*>(dosb + rq + 16 * s);
            fv[i] = *reinterpret_cast<const op_t*>(vbase + 16 * s);
        };
        if constexpr (MFA_BWD_PREFETCH) {
            ld_sdp(0, 0);
            static_for<DS>([&](auto sc) __attribute__((always_inline)) {
                constexpr int s = decltype(sc)::value;
                if constexpr (s + 1 < DS) ld_sdp(s + 1, (s + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
                sacc = O::mfma(fq[s & 1], fk[s & 1], sacc);
                dpacc = O::mfma(fd[s & 1], fv[s & 1], dpacc);
                __builtin_amdgcn_sched_barrier(0);
            });
        } else {
#pragma unroll
            for (int s = 0; s < DS; ++s) {
                ld_sdp(s, 0);
                sacc = O::mfma(fq[0], fk[0], sacc);
                dpacc = O::mfma(fd[0], fv[0], dpacc);
            }
        }
        // the first dV/dK fragments, read before the vector work below
        op_t fdo[2], fqt[2];
        auto ld_dvdk = [&](int idx, int i) __attribute__((always_inline)) {
            const int o = rt + 2560 * (idx / DB) + 32 * (idx % DB);
            fdo[i] = O::load_tr_rows(dosb + o, dosb + o + 1296);
            fqt[i] = O::load_tr_rows(qsb + o, qsb + o + 1296);
        };
        if constexpr (MFA_BWD_PREFETCH) ld_dvdk(0, 0);
        // P and dS rounded to 16 bits (register r is query qs0 + acc_row(r) +
        // 4*half); sub-blocks whose 32 x 32 pairs are all valid skip the masks
        uint32_t pw[8], dw[8];
        const bool full = qs0 + 32 <= Lq && key_lo(f, qs0 + 31 + dq) <= wk0 && key_hi(f, qs0 + dq, Lk) >= wk0 + 31;
        auto probs = [&](auto masked_tag) {
            constexpr bool MASKED = decltype(masked_tag)::value;
            // ALiBi distance center - key of register r: this lane's base plus
            // the register's row offset, exact in fp32 below 2^24 (formed in
            // each path: the pin keeps the per-register values from being
            // hoisted above the branch)
            float dist0 = (float)(qs0 + 4 * half + dq - key);
            asm volatile("" : "+v"(dist0));
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 l4 = *reinterpret_cast<const float4*>(lsb + 8 * g + 4 * half);
                const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
                float p[4], ds[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * g + i;
                    const int q = qs0 + acc_row(r) + 4 * half;
                    const int center = q + dq;
                    float dcap;
                    const float x = transform<BIAS>(f, sacc[r], slope, dist0 + (float)acc_row(r), dcap);
                    const float pe = fast_exp2(fmaf(x, c, -lv[i]));
                    bool ok = true;
                    if constexpr (MASKED)
                        ok = (key <= key_hi(f, center, Lk)) & (key >= key_lo(f, center)) & (q < Lq);
                    p[i] = ok ? pe : 0.f;
                    ds[i] = p[i] * dpacc[r];
                    if constexpr (BIAS) ds[i] *= dcap;
                }
                pw[2 * g] = O::pack(p[0], p[1]);
                pw[2 * g + 1] = O::pack(p[2], p[3]);
                dw[2 * g] = O::pack(ds[0], ds[1]);
                dw[2 * g + 1] = O::pack(ds[2], ds[3]);
            }
        };
        if (full)
            probs(std::false_type{});
        else
            probs(std::true_type{});
        // dV^T += dO^T P, dK^T += Q^T dS (k-slots = query rows of accumulator
        // registers 8*st..8*st+7)
        if constexpr (MFA_BWD_PREFETCH) {
            static_for<2 * DB>([&](auto ic) __attribute__((always_inline)) {
                constexpr int idx = decltype(ic)::value, st = idx / DB, db = idx % DB;
                if constexpr (idx + 1 < 2 * DB) ld_dvdk(idx + 1, (idx + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
                const u32x4_t pv = {pw[4 * st], pw[4 * st + 1], pw[4 * st + 2], pw[4 * st + 3]};
                const u32x4_t dsv = {dw[4 * st], dw[4 * st + 1], dw[4 * st + 2], dw[4 * st + 3]};
                dva[db] = O::mfma(fdo[idx & 1], __builtin_bit_cast(op_t, pv), dva[db]);
                dka[db] = O::mfma(fqt[idx & 1], __builtin_bit_cast(op_t, dsv), dka[db]);
                __builtin_amdgcn_sched_barrier(0);
            });
        } else {
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const u32x4_t pv = {pw[4 * st], pw[4 * st + 1], pw[4 * st + 2], pw[4 * st + 3]};
                const u32x4_t dsv = {dw[4 * st], dw[4 * st + 1], dw[4 * st + 2], dw[4 * st + 3]};
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    ld_dvdk(st * DB + db, 0);
                    dva[db] = O::mfma(fdo[0], __builtin_bit_cast(op_t, pv), dva[db]);
                    dka[db] = O::mfma(fqt[0], __builtin_bit_cast(op_t, dsv), dka[db]);
                }
            }
        }
        if (step + 1 < nsteps) swrite(buf ^ 1);  // the other stage was last read before the previous barrier
        __syncthreads();
    }
    // pair sums: wavefront w + 4 hands its partials to wavefront w through
    // LDS (every wavefront has passed the last barrier, so K/V are dead)
    float* red = reinterpret_cast<float*>(kv_s) + kw * (DB * 16 * 64) + lane;
    auto pair_sum = [&](f32x16_t(&acc)[DB]) __attribute__((always_inline)) {
        if (sb == 1) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) red[(db * 16 + r) * 64] = acc[db][r];
        }
        __syncthreads();
        if (sb == 0) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[db][r] += red[(db * 16 + r) * 64];
        }
        __syncthreads();
    };
    pair_sum(dka);
    pair_sum(dva);
    if (sb == 0 && key < Lk) {
        if (a.G > 1) {  // this group's partial sums, unscaled, fp32
            const int64_t orow = ((int64_t)grp * a.Ukv + unit) * f.Lk + key;
            store_rows<DB>(reinterpret_cast<char*>(a.ws_dk + orow * a.ws_ld), 0, D, true, IS_BF16, dka, 1.f, half);
            store_rows<DB>(reinterpret_cast<char*>(a.ws_dv + orow * a.ws_ld), 0, D, true, IS_BF16, dva, 1.f, half);
        } else {
            const bool f32o = a.grad_f32 != 0;
            const int ges = f32o ? 4 : 2;
            store_rows<DB>(kv.dk + (int64_t)key * a.dks * ges, 0, D, f32o, IS_BF16, dka, f.scale, half);
            store_rows<DB>(kv.dv + (int64_t)key * a.dvs * ges, 0, D, f32o, IS_BF16, dva, 1.f, half);
        }
    }
}

// Sum of the G head-group partials of dK / dV in group order (deterministic),
// scaled (dK) and stored in the gradient dtype: 4 elements per thread.
template <bool IS_BF16>
__global__ void __launch_bounds__(kBThreads) mfa_bwd_dkdv_sum_kernel(BArgs a) {
    const KArgs& f = a.f;
    const int per_row = f.D / 4;
    const int64_t idx = (int64_t)blockIdx.x * kBThreads + threadIdx.x;
    const int64_t rows = (int64_t)a.Ukv * f.Lk;
    if (idx >= rows * per_row) return;
    const int64_t r = idx / per_row;
    const int d = (int)(idx - r * per_row) * 4;
    const int unit = (int)(r / f.Lk), key = (int)(r - (int64_t)unit * f.Lk);
    const int b = unit / f.Hkv, hkv = unit - b * f.Hkv;
    const KView kv = k_view(a, b, hkv);
    if (key >= kv.Lk) return;
    float4 sk = make_float4(0.f, 0.f, 0.f, 0.f), sv = sk;
    for (int g = 0; g < a.G; ++g) {
        const int64_t off = (((int64_t)g * a.Ukv + unit) * f.Lk + key) * a.ws_ld + d;
        const float4 x = *reinterpret_cast<const float4*>(a.ws_dk + off);
        const float4 y = *reinterpret_cast<const float4*>(a.ws_dv + off);
        sk.x += x.x; sk.y += x.y; sk.z += x.z; sk.w += x.w;
        sv.x += y.x; sv.y += y.y; sv.z += y.z; sv.w += y.w;
    }
    const float sc = f.scale;
    const float k4[4] = {sk.x * sc, sk.y * sc, sk.z * sc, sk.w * sc};
    const float v4[4] = {sv.x, sv.y, sv.z, sv.w};
    if (a.grad_f32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(kv.dk) + (int64_t)key * a.dks + d) =
            make_float4(k4[0], k4[1], k4[2], k4[3]);
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(kv.dv) + (int64_t)key * a.dvs + d) =
            make_float4(v4[0], v4[1], v4[2], v4[3]);
    } else {
        const uint32_t kw0 = Ops<IS_BF16>::pack(k4[0], k4[1]), kw1 = Ops<IS_BF16>::pack(k4[2], k4[3]);
        const uint32_t vw0 = Ops<IS_BF16>::pack(v4[0], v4[1]), vw1 = Ops<IS_BF16>::pack(v4[2], v4[3]);
        *reinterpret_cast<u32x2_t*>(kv.dk + ((int64_t)key * a.dks + d) * 2) = u32x2_t{kw0, kw1};
        *reinterpret_cast<u32x2_t*>(kv.dv + ((int64_t)key * a.dvs + d) * 2) = u32x2_t{vw0, vw1};
    }
}

// ----------------------------------------------------------------------------
// dQ: workgroup = 128 query rows of one (sequence, query head), 32 per wavefront.
template <int DP, bool IS_BF16, bool BIAS>
__global__ void __launch_bounds__(kBThreads) __attribute__((amdgpu_waves_per_eu(1)))
mfa_bwd_dq_kernel(BArgs a) {
    typedef Ops<IS_BF16> O;
    typedef typename O::op_t op_t;
    constexpr int DS = DP / 16, DB = DP / 32;
    constexpr int NKB = MFA_BWD_DQ_NKB, BN = 32 * NKB;  // keys per block
    static_assert(BN <= 128, "the host bounds a staged block's byte span for 128 rows");
    constexpr int KST = DP + 8;
    constexpr int CPR = DP / 8;
    constexpr int SCH = (BN * CPR + kBThreads - 1) / kBThreads;  // staged chunks per thread and tensor
    __shared__ __attribute__((aligned(16))) uint16_t k_s[2][BN * KST];
    __shared__ __attribute__((aligned(16))) uint16_t v_s[2][BN * KST];

    const KArgs& f = a.f;
    const int bid = blockIdx.x;
    const int tt = bid / f.U, unit = bid - tt * f.U;
    const int tile = a.T - 1 - tt;  // heaviest (causal: last) query tiles first
    const int b = unit / f.Hq, hq = unit - b * f.Hq;
    const int hkv = hq / (f.Hq / f.Hkv);
    const QView qv = q_view(a, b, hq);
    const KView kv = k_view(a, b, hkv);
    const int Lq = qv.Lq, Lk = kv.Lk, D = f.D;
    const int q0 = tile * 128;
    if (q0 >= Lq) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int dq = Lk - Lq;
    const int wq0 = q0 + wave * 32;      // first query row of this wavefront
    const int q = wq0 + l32;             // this lane's query
    const bool qin = q < Lq;

    // Q and dO rows as B operands (k-slots d = 16*s + 8*half + 0..7)
    op_t qf[DS], dof[DS];
#pragma unroll
    for (int s = 0; s < DS; ++s) {
        const int d = 16 * s + 8 * half;
        u32x4_t qq = {0, 0, 0, 0}, gg = {0, 0, 0, 0};
        if (qin && d < D) {
            qq = *reinterpret_cast<const u32x4_t*>(qv.q + ((int64_t)q * f.qs + d) * 2);
            gg = *reinterpret_cast<const u32x4_t*>(qv.dout + ((int64_t)q * a.dos + d) * 2);
        }
        qf[s] = __builtin_bit_cast(op_t, qq);
        dof[s] = __builtin_bit_cast(op_t, gg);
    }
    const float lse2 = qin ? lse2_of(qv.lse[q]) : INFINITY;
    const float dsum = qin ? qv.dsum[q] : 0.f;
    constexpr bool DFOLD = DP <= 64;  // registers allow the -Dsum vector
    f32x16_t negd;
#pragma unroll
    for (int r = 0; r < 16; ++r) negd[r] = -dsum;
    const int center = q + dq;
    const int lo = key_lo(f, center), hi = key_hi(f, center, Lk);
    const float slope = BIAS && f.alibi ? f.alibi[b * f.alibi_bstride + hq] : 0.f;
    const float c = BIAS ? kLog2e : f.scale_log2;
    f32x16_t dqa[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dqa[db][r] = 0.f;

    // key blocks any row of the workgroup can see
    const int qlast = min(q0 + 128, Lq) - 1;
    const int klo = key_lo(f, q0 + dq);
    const int khi = key_hi(f, qlast + dq, Lk);
    const int jbeg = (klo / BN) * BN;
    const int nblk = khi >= klo ? (khi - jbeg) / BN + 1 : 0;
    // buffer-load staging as in the dK/dV kernel (rows past the sequence read zero)
    u32x4_t sk[SCH], sv2[SCH];
    uint32_t koff[SCH], voff[SCH];
    int soff[SCH];
#pragma unroll
    for (int i = 0; i < SCH; ++i) {
        const int cc = tid + kBThreads * i;
        const int row = cc / CPR, col = (cc % CPR) * 8;
        const bool in = cc < BN * CPR && col < D;
        koff[i] = in ? (uint32_t)(((int64_t)row * f.ks + col) * 2) : 0x80000000u;
        voff[i] = in ? (uint32_t)(((int64_t)row * f.vs + col) * 2) : 0x80000000u;
        soff[i] = (MFA_BWD_PERM ? prow(row) : row) * KST + col;
    }
    auto gload = [&](int u) {
        const int j = jbeg + u * BN;
        const int rm1 = min(Lk - j, BN) - 1;  // j < Lk
        const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(kv.k + (int64_t)j * f.ks * 2), (short)0, (int)(((int64_t)rm1 * f.ks + D) * 2), kBufferDword3);
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(kv.v + (int64_t)j * f.vs * 2), (short)0, (int)(((int64_t)rm1 * f.vs + D) * 2), kBufferDword3);
#pragma unroll
        for (int i = 0; i < SCH; ++i) {
            sk[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, koff[i], 0, 0);
            sv2[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, voff[i], 0, 0);
        }
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int i = 0; i < SCH; ++i) {
            if (SCH * kBThreads == BN * CPR || tid + kBThreads * i < BN * CPR) {
                *reinterpret_cast<u32x4_t*>(k_s[buf] + soff[i]) = sk[i];
                *reinterpret_cast<u32x4_t*>(v_s[buf] + soff[i]) = sv2[i];
            }
        }
    };
    if (nblk > 0) {
        gload(0);
        swrite(0);
    }
    __syncthreads();
    for (int u = 0; u < nblk; ++u) {
        const int j = jbeg + u * BN;
        const int buf = u & 1;
        if (u + 1 < nblk) gload(u + 1);  // in flight during this block's MFMAs
        const uint16_t* ksb = k_s[buf];
        const uint16_t* vsb = v_s[buf];
        // one 32-key block at a time: S^T, dP^T, dS^T, then its dQ products
        // (operand reads pipelined one MFMA pair ahead, as in the dK/dV kernel)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            // S^T = K Q^T and dP^T = V dO^T (lane = query, registers = keys)
            // (at DP <= 64 dP^T starts from -Dsum, a register vector the first
            // MFMA reads as its C operand, so the accumulator ends as dP - Dsum)
            f32x16_t sacc, dpacc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
            if constexpr (DFOLD)
                dpacc = negd;
            else
#pragma unroll
                for (int r = 0; r < 16; ++r) dpacc[r] = 0.f;
            op_t fk[2], fv[2];
            auto ld_kv = [&](int s, int i) __attribute__((always_inline)) {
                const int krow = 32 * kb + (MFA_BWD_PERM ? prow(l32) : l32);
                fk[i] = *reinterpret_cast<const op_t*>(ksb + krow * KST + 16 * s + 8 * half);
                fv[i] = *reinterpret_cast<const op_t*>(vsb + krow * KST + 16 * s + 8 * half);
            };
            if constexpr (MFA_BWD_PREFETCH) {
                ld_kv(0, 0);
                static_for<DS>([&](auto sc) __attribute__((always_inline)) {
                    constexpr int s = decltype(sc)::value;
                    if constexpr (s + 1 < DS) ld_kv(s + 1, (s + 1) & 1);
                    __builtin_amdgcn_sched_barrier(0);
                    sacc = O::mfma(fk[s & 1], qf[s], sacc);
                    dpacc = O::mfma(fv[s & 1], dof[s], dpacc);
                    __builtin_amdgcn_sched_barrier(0);
                });
            } else {
#pragma unroll
                for (int s = 0; s < DS; ++s) {
                    ld_kv(s, 0);
                    sacc = O::mfma(fk[0], qf[s], sacc);
                    dpacc = O::mfma(fv[0], dof[s], dpacc);
                }
            }
            // the first K^T fragment, read before the vector work below
            op_t fkt[2];
            auto ld_kt = [&](int idx, int i) __attribute__((always_inline)) {
                fkt[i] = MFA_BWD_PERM ? O::load_tr_perm(ksb, KST, 32 * kb + 16 * (idx / DB), 32 * (idx % DB), lane)
                                      : O::load_tr(ksb, KST, 32 * kb + 16 * (idx / DB), 32 * (idx % DB), lane);
            };
            if constexpr (MFA_BWD_PREFETCH) ld_kt(0, 0);
            // tiles whose 32 x 32 pairs are all valid skip the masks
            const int kk0 = j + 32 * kb;
            const bool full = wq0 + 31 < Lq && key_lo(f, wq0 + 31 + dq) <= kk0 && key_hi(f, wq0 + dq, Lk) >= kk0 + 31;
            uint32_t dw[8];
            auto dsrow = [&](auto masked_tag) {
                constexpr bool MASKED = decltype(masked_tag)::value;
                // ALiBi distance center - key of register r: this lane's base
                // minus the register's key offset, exact in fp32 below 2^24
                // (formed in each path: the pin keeps the compiler from
                // hoisting the 16 per-register values above the branch)
                float dist0 = (float)(center - kk0 - 4 * half);
                asm volatile("" : "+v"(dist0));
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    float ds2[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const int key = kk0 + acc_row(r + i) + 4 * half;
                        float dcap;
                        const float x = transform<BIAS>(f, sacc[r + i], slope, dist0 - (float)acc_row(r + i), dcap);
                        const float pe = fast_exp2(fmaf(x, c, -lse2));
                        bool ok = true;
                        if constexpr (MASKED) ok = (key >= lo) & (key <= hi) & qin;
                        const float p = ok ? pe : 0.f;
                        ds2[i] = DFOLD ? p * dpacc[r + i] : p * (dpacc[r + i] - dsum);
                        if constexpr (BIAS) ds2[i] *= dcap;
                    }
                    dw[r / 2] = O::pack(ds2[0], ds2[1]);
                }
            };
            if (full)
                dsrow(std::false_type{});
            else
                dsrow(std::true_type{});
            // dQ^T += K^T dS^T (k-slots = keys of accumulator registers 8*st..8*st+7)
            if constexpr (MFA_BWD_PREFETCH) {
                static_for<2 * DB>([&](auto ic) __attribute__((always_inline)) {
                    constexpr int idx = decltype(ic)::value, st = idx / DB, db = idx % DB;
                    if constexpr (idx + 1 < 2 * DB) ld_kt(idx + 1, (idx + 1) & 1);
                    __builtin_amdgcn_sched_barrier(0);
                    const u32x4_t dsv = {dw[4 * st], dw[4 * st + 1], dw[4 * st + 2], dw[4 * st + 3]};
                    dqa[db] = O::mfma(fkt[idx & 1], __builtin_bit_cast(op_t, dsv), dqa[db]);
                    __builtin_amdgcn_sched_barrier(0);
                });
            } else {
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const u32x4_t dsv = {dw[4 * st], dw[4 * st + 1], dw[4 * st + 2], dw[4 * st + 3]};
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        ld_kt(st * DB + db, 0);
                        dqa[db] = O::mfma(fkt[0], __builtin_bit_cast(op_t, dsv), dqa[db]);
                    }
                }
            }
        }
        if (u + 1 < nblk) swrite(buf ^ 1);
        __syncthreads();
    }
    if (qin) {
        const bool f32o = a.grad_f32 != 0;
        const int ges = f32o ? 4 : 2;
        store_rows<DB>(qv.dq + (int64_t)q * a.dqs * ges, 0, D, f32o, IS_BF16, dqa, f.scale, half);
    }
}

// ----------------------------------------------------------------------------
// fp32 backward: fp32 q, k, v, o and dO in, fp32 dq, dk and dv out.  The same
// decomposition as the 16-bit kernels (Dsum; dK/dV for a block of keys of one
// (sequence, K/V head), walking every query block of its head group that
// sees them; dQ for a block of query rows, walking the key blocks they see),
// with fp32 products on the vector ALU over LDS tiles and the fp32 forward's
// score transform (precise tanh under soft-cap): the gradients of an fp32
// forward, computed in fp32 end to end.  Tiles: 32 query rows x 64 keys;
// thread t computes the scores of rows 2*(t/16), +1 and keys 4*(t%16)..+3.

constexpr int kB32Rows = 32;              // query rows of a tile
constexpr int kB32Keys = 64;              // keys of a tile
constexpr int kB32KT = kB32Keys + 4;      // row stride (floats) of transposed K/V tiles

// Per (sequence, query head) / (sequence, K/V head) rows of fp32 tensors
// (element offsets, as q_view / k_view).
struct QView32 {
    const float* q;
    const float* dout;
    const float* o;
    float* dq;
    const float* lse;
    float* dsum;
    int Lq, Lk;
};
__device__ __forceinline__ QView32 q_view32(const BArgs& a, int b, int hq) {
    const KArgs& f = a.f;
    QView32 s;
    int64_t qs = 0, qb = 0;
    if (f.cu_q) {
        const int q0 = f.cu_q[b];
        s.Lq = f.cu_q[b + 1] - q0;
        s.Lk = f.cu_k[b + 1] - f.cu_k[b];
        qs = q0;
        s.lse = f.lse + (int64_t)hq * f.lse_h + q0;
    } else {
        s.Lq = f.Lq;
        s.Lk = f.Lk;
        qb = b;
        s.lse = f.lse + (int64_t)b * f.lse_b + (int64_t)hq * f.lse_h;
    }
    s.q = reinterpret_cast<const float*>(f.q) + (qb * f.qb + qs * f.qs + (int64_t)hq * f.qh);
    s.o = reinterpret_cast<const float*>(f.o) + (qb * f.ob + qs * f.os + (int64_t)hq * f.oh);
    s.dout = reinterpret_cast<const float*>(a.dout) + (qb * a.dob + qs * a.dos + (int64_t)hq * a.doh);
    s.dq = reinterpret_cast<float*>(a.dq) + (qb * a.dqb + qs * a.dqs + (int64_t)hq * a.dqh);
    s.dsum = a.dsum + ((int64_t)b * f.Hq + hq) * f.Lq;
    return s;
}
struct KView32 {
    const float* k;
    const float* v;
    float* dk;
    float* dv;
    int Lk;
};
__device__ __forceinline__ KView32 k_view32(const BArgs& a, int b, int hkv) {
    const KArgs& f = a.f;
    KView32 s;
    int64_t ks = 0, kb = 0;
    if (f.cu_k) {
        ks = f.cu_k[b];
        s.Lk = f.cu_k[b + 1] - f.cu_k[b];
    } else {
        kb = b;
        s.Lk = f.Lk;
    }
    s.k = reinterpret_cast<const float*>(f.k) + (kb * f.kb + ks * f.ks + (int64_t)hkv * f.kh);
    s.v = reinterpret_cast<const float*>(f.v) + (kb * f.vb + ks * f.vs + (int64_t)hkv * f.vh);
    s.dk = reinterpret_cast<float*>(a.dk) + (kb * a.dkb + ks * a.dks + (int64_t)hkv * a.dkh);
    s.dv = reinterpret_cast<float*>(a.dv) + (kb * a.dvb + ks * a.dvs + (int64_t)hkv * a.dvh);
    return s;
}

// Rows [0, NROWS) of an fp32 [rows, D] tile (row stride `st` floats) into
// LDS, transposed (t[d * TS + row]) and, with ROWS, also row-major
// (r[row * (DP + 4) + d]).  Rows >= `valid` and columns >= D read as 0.
// Every load of a thread is issued before its LDS stores.
template <int DP, int NROWS, int TS, bool ROWS>
__device__ __forceinline__ void stage32(const float* src, int64_t st, int valid, int D, float* t, float* r, int tid) {
    constexpr int C4 = DP / 4;  // float4 chunks per row
    constexpr int N = (NROWS * C4 + kBThreads - 1) / kBThreads;
    float4 v[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int cc = tid + kBThreads * i;
        const int row = cc / C4, col = (cc % C4) * 4;
        v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (cc < NROWS * C4 && row < valid && col < D)
            v[i] = *reinterpret_cast<const float4*>(src + (int64_t)row * st + col);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int cc = tid + kBThreads * i;
        if (N * kBThreads == NROWS * C4 || cc < NROWS * C4) {
            const int row = cc / C4, col = (cc % C4) * 4;
            t[(col + 0) * TS + row] = v[i].x;
            t[(col + 1) * TS + row] = v[i].y;
            t[(col + 2) * TS + row] = v[i].z;
            t[(col + 3) * TS + row] = v[i].w;
            if constexpr (ROWS) *reinterpret_cast<float4*>(r + row * (DP + 4) + col) = v[i];
        }
    }
}

// S = Q K^T and dP = dO V^T of one 32 x 64 tile from transposed LDS tiles
// (q / dO: [DP][32], k / v: [DP][kB32KT]): rows r, r+1, keys c..c+3.
template <int DP>
__device__ __forceinline__ void tile_products32(const float* qt, const float* dot, const float* kt, const float* vt,
                                                int r, int c, float (&s)[2][4], float (&g)[2][4]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) s[i][j] = g[i][j] = 0.f;
#pragma unroll 4
    for (int d = 0; d < DP; ++d) {
        const float2 qa = *reinterpret_cast<const float2*>(qt + d * kB32Rows + r);
        const float2 ga = *reinterpret_cast<const float2*>(dot + d * kB32Rows + r);
        const float4 kb = *reinterpret_cast<const float4*>(kt + d * kB32KT + c);
        const float4 vb = *reinterpret_cast<const float4*>(vt + d * kB32KT + c);
        const float kk[4] = {kb.x, kb.y, kb.z, kb.w}, vv[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[0][j] = fmaf(qa.x, kk[j], s[0][j]);
            s[1][j] = fmaf(qa.y, kk[j], s[1][j]);
            g[0][j] = fmaf(ga.x, vv[j], g[0][j]);
            g[1][j] = fmaf(ga.y, vv[j], g[1][j]);
        }
    }
}

// One query row's data for the tile: exp2-domain lse, Dsum, center and
// valid key interval (hi = -1 for a row past the sequence).
struct Row32 {
    float lse2, dsum;
    int center, lo, hi;
};
__device__ __forceinline__ Row32 row32(const KArgs& f, const QView32& qv, int q, int dq, int Lk) {
    Row32 w;
    const bool in = q < qv.Lq;
    w.lse2 = in ? lse2_of(qv.lse[q]) : INFINITY;
    w.dsum = in ? qv.dsum[q] : 0.f;
    w.center = q + dq;
    w.lo = key_lo(f, w.center);
    w.hi = in ? key_hi(f, w.center, Lk) : -1;
    return w;
}

// P and dS * d score / d (q.k) of one (row, key) pair from s = q.k and dP:
// score = scale*s, soft-cap (precise tanh), ALiBi; P = exp(score - lse).
__device__ __forceinline__ void pair32(const KArgs& f, const Row32& w, float slope, int key, float s, float dp,
                                       float& p, float& ds) {
    float x = s * f.scale, dx = f.scale;
    if (f.softcap > 0.f) {
        const float t = precise_tanh(__fdiv_rn(x, f.softcap));
        x = f.softcap * t;
        dx *= 1.f - t * t;
    }
    if (f.alibi) x = fmaf(-slope, fabsf((float)(w.center - key)), x);
    const bool valid = key >= w.lo && key <= w.hi;
    p = valid ? fast_exp2(fmaf(x, kLog2e, -w.lse2)) : 0.f;
    ds = p * (dp - w.dsum) * dx;
}

// Dsum = rowsum(dO * O) - dlse in fp32: 16 lanes per row, 8 elements per lane.
__global__ void __launch_bounds__(kBThreads) mfa_bwd32_dsum_kernel(BArgs a) {
    const int bid = blockIdx.x;
    const int unit = bid / a.T, tile = bid - unit * a.T;
    const int b = unit / a.f.Hq, hq = unit - b * a.f.Hq;
    const QView32 qv = q_view32(a, b, hq);
    const int row = tile * 16 + (threadIdx.x >> 4), sub = threadIdx.x & 15;
    float acc = 0.f;
    const int d0 = sub * 8;
    if (row < qv.Lq && d0 < a.f.D) {  // (D is a multiple of 8)
#pragma unroll
        for (int e = 0; e < 8; e += 4) {
            const float4 o = *reinterpret_cast<const float4*>(qv.o + (int64_t)row * a.f.os + d0 + e);
            const float4 g = *reinterpret_cast<const float4*>(qv.dout + (int64_t)row * a.dos + d0 + e);
            acc = fmaf(o.x, g.x, acc);
            acc = fmaf(o.y, g.y, acc);
            acc = fmaf(o.z, g.z, acc);
            acc = fmaf(o.w, g.w, acc);
        }
    }
    acc += __shfl_xor(acc, 8);
    acc += __shfl_xor(acc, 4);
    acc += __shfl_xor(acc, 2);
    acc += __shfl_xor(acc, 1);
    if (sub == 0 && row < qv.Lq) {
        if (a.dlse) {
            const float* dl = a.dlse + (qv.lse - a.f.lse);
            acc -= dl[row];
        }
        qv.dsum[row] = acc;
    }
}

// dQ of 32 query rows: dQ = sum over key blocks of dS' K (dS' = dS * d score
// / d(q.k)), K staged transposed (for S) and row-major (for the product).
template <int DP>
__global__ void __launch_bounds__(kBThreads) mfa_bwd32_dq_kernel(BArgs a) {
    const KArgs& f = a.f;
    const int unit = blockIdx.x / a.T, tile = blockIdx.x - unit * a.T;
    const int b = unit / f.Hq, hq = unit - b * f.Hq;
    const QView32 qv = q_view32(a, b, hq);
    const KView32 kv = k_view32(a, b, hq / (f.Hq / f.Hkv));
    const int Lq = qv.Lq, Lk = kv.Lk, D = f.D;
    const int q0 = tile * kB32Rows;
    if (q0 >= Lq) return;
    const int tid = threadIdx.x;
    const int r = 2 * (tid >> 4), c = 4 * (tid & 15);
    constexpr int DC = DP / 16;  // dQ columns per thread
    const int d0 = (tid & 15) * DC;
    const int dq = Lk - Lq;
    const int nrow = min(kB32Rows, Lq - q0);

    __shared__ __attribute__((aligned(16))) float qt[DP * kB32Rows];
    __shared__ __attribute__((aligned(16))) float dot[DP * kB32Rows];
    __shared__ __attribute__((aligned(16))) float kt[DP * kB32KT];
    __shared__ __attribute__((aligned(16))) float vt[DP * kB32KT];
    __shared__ __attribute__((aligned(16))) float kr[kB32Keys * (DP + 4)];
    __shared__ __attribute__((aligned(16))) float dst[kB32Keys * kB32Rows];  // dS'^T [key][row]

    stage32<DP, kB32Rows, kB32Rows, false>(qv.q + (int64_t)q0 * f.qs, f.qs, nrow, D, qt, nullptr, tid);
    stage32<DP, kB32Rows, kB32Rows, false>(qv.dout + (int64_t)q0 * a.dos, a.dos, nrow, D, dot, nullptr, tid);
    const Row32 w0 = row32(f, qv, q0 + r, dq, Lk), w1 = row32(f, qv, q0 + r + 1, dq, Lk);
    const float slope = f.alibi ? f.alibi[b * f.alibi_bstride + hq] : 0.f;

    float acc[2][DC];
#pragma unroll
    for (int e = 0; e < DC; ++e) acc[0][e] = acc[1][e] = 0.f;
    // key blocks any row of the tile sees (the bounds are monotone in the row)
    const int klo = key_lo(f, q0 + dq), khi = key_hi(f, q0 + nrow - 1 + dq, Lk);
    for (int j0 = (klo / kB32Keys) * kB32Keys; j0 <= khi; j0 += kB32Keys) {
        const int nk = min(kB32Keys, Lk - j0);
        __syncthreads();  // (the previous block's LDS reads are done; the Q tiles are visible)
        stage32<DP, kB32Keys, kB32KT, true>(kv.k + (int64_t)j0 * f.ks, f.ks, nk, D, kt, kr, tid);
        stage32<DP, kB32Keys, kB32KT, false>(kv.v + (int64_t)j0 * f.vs, f.vs, nk, D, vt, nullptr, tid);
        __syncthreads();
        float s[2][4], g[2][4];
        tile_products32<DP>(qt, dot, kt, vt, r, c, s, g);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float p, ds0, ds1;
            pair32(f, w0, slope, j0 + c + j, s[0][j], g[0][j], p, ds0);
            pair32(f, w1, slope, j0 + c + j, s[1][j], g[1][j], p, ds1);
            *reinterpret_cast<float2*>(dst + (c + j) * kB32Rows + r) = make_float2(ds0, ds1);
        }
        __syncthreads();
#pragma unroll 4
        for (int j = 0; j < kB32Keys; ++j) {
            const float2 gr = *reinterpret_cast<const float2*>(dst + j * kB32Rows + r);
            const float* kp = kr + j * (DP + 4) + d0;
#pragma unroll
            for (int e = 0; e < DC; e += 2) {
                const float2 kk = *reinterpret_cast<const float2*>(kp + e);
                acc[0][e] = fmaf(gr.x, kk.x, acc[0][e]);
                acc[0][e + 1] = fmaf(gr.x, kk.y, acc[0][e + 1]);
                acc[1][e] = fmaf(gr.y, kk.x, acc[1][e]);
                acc[1][e + 1] = fmaf(gr.y, kk.y, acc[1][e + 1]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = q0 + r + i;
        if (q < Lq) {
#pragma unroll
            for (int e = 0; e < DC; ++e)
                if (d0 + e < D) qv.dq[(int64_t)q * a.dqs + d0 + e] = acc[i][e];
        }
    }
}

// dK and dV of 64 keys of one (sequence, K/V head): every query block of
// every query head of the group that sees the keys adds P^T dO to dV and
// dS'^T Q to dK (in a fixed order: the result does not depend on scheduling).
template <int DP>
__global__ void __launch_bounds__(kBThreads) mfa_bwd32_dkdv_kernel(BArgs a) {
    const KArgs& f = a.f;
    const int ukv = blockIdx.x / a.T, ktile = blockIdx.x - ukv * a.T;
    const int b = ukv / f.Hkv, hkv = ukv - b * f.Hkv;
    const KView32 kv = k_view32(a, b, hkv);
    const int Lk = kv.Lk, D = f.D;
    const int k0 = ktile * kB32Keys;
    if (k0 >= Lk) return;
    const int nk = min(kB32Keys, Lk - k0);
    const int tid = threadIdx.x;
    const int r = 2 * (tid >> 4), c = 4 * (tid & 15);  // score tile: rows r, r+1; keys c..c+3
    constexpr int DC = DP / 16;
    const int kk0 = 4 * (tid >> 4), d0 = (tid & 15) * DC;  // dK/dV tile: keys kk0..kk0+3, columns d0..

    __shared__ __attribute__((aligned(16))) float kt[DP * kB32KT];
    __shared__ __attribute__((aligned(16))) float vt[DP * kB32KT];
    __shared__ __attribute__((aligned(16))) float qt[DP * kB32Rows];
    __shared__ __attribute__((aligned(16))) float dot[DP * kB32Rows];
    __shared__ __attribute__((aligned(16))) float qr[kB32Rows * (DP + 4)];
    __shared__ __attribute__((aligned(16))) float dor[kB32Rows * (DP + 4)];
    __shared__ __attribute__((aligned(16))) float ps[kB32Rows * kB32Keys];  // P [row][key]
    __shared__ __attribute__((aligned(16))) float gs[kB32Rows * kB32Keys];  // dS' [row][key]

    stage32<DP, kB32Keys, kB32KT, false>(kv.k + (int64_t)k0 * f.ks, f.ks, nk, D, kt, nullptr, tid);
    stage32<DP, kB32Keys, kB32KT, false>(kv.v + (int64_t)k0 * f.vs, f.vs, nk, D, vt, nullptr, tid);

    float dk[4][DC], dv[4][DC];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < DC; ++e) dk[j][e] = dv[j][e] = 0.f;
    const int R = f.Hq / f.Hkv;
    const int Lq = f.cu_q ? f.cu_q[b + 1] - f.cu_q[b] : f.Lq;
    const int dq = Lk - Lq;
    const int k1 = k0 + nk - 1;
    for (int rr = 0; rr < R; ++rr) {
        const int hq = hkv * R + rr;
        const QView32 qv = q_view32(a, b, hq);
        const float slope = f.alibi ? f.alibi[b * f.alibi_bstride + hq] : 0.f;
        for (int q0 = 0; q0 < Lq; q0 += kB32Rows) {
            const int nrow = min(kB32Rows, Lq - q0);
            // (no row of the block sees a key of the tile: the bounds are monotone in the row)
            if (key_hi(f, q0 + nrow - 1 + dq, Lk) < k0 || key_lo(f, q0 + dq) > k1) continue;
            __syncthreads();  // (the previous block's LDS reads are done; the K/V tiles are visible)
            stage32<DP, kB32Rows, kB32Rows, true>(qv.q + (int64_t)q0 * f.qs, f.qs, nrow, D, qt, qr, tid);
            stage32<DP, kB32Rows, kB32Rows, true>(qv.dout + (int64_t)q0 * a.dos, a.dos, nrow, D, dot, dor, tid);
            const Row32 w0 = row32(f, qv, q0 + r, dq, Lk), w1 = row32(f, qv, q0 + r + 1, dq, Lk);
            __syncthreads();
            float s[2][4], g[2][4];
            tile_products32<DP>(qt, dot, kt, vt, r, c, s, g);
            float p0[4], p1[4], g0[4], g1[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                pair32(f, w0, slope, k0 + c + j, s[0][j], g[0][j], p0[j], g0[j]);
                pair32(f, w1, slope, k0 + c + j, s[1][j], g[1][j], p1[j], g1[j]);
            }
            *reinterpret_cast<float4*>(ps + r * kB32Keys + c) = make_float4(p0[0], p0[1], p0[2], p0[3]);
            *reinterpret_cast<float4*>(ps + (r + 1) * kB32Keys + c) = make_float4(p1[0], p1[1], p1[2], p1[3]);
            *reinterpret_cast<float4*>(gs + r * kB32Keys + c) = make_float4(g0[0], g0[1], g0[2], g0[3]);
            *reinterpret_cast<float4*>(gs + (r + 1) * kB32Keys + c) = make_float4(g1[0], g1[1], g1[2], g1[3]);
            __syncthreads();
#pragma unroll 2
            for (int i = 0; i < nrow; ++i) {
                const float4 pv = *reinterpret_cast<const float4*>(ps + i * kB32Keys + kk0);
                const float4 gv = *reinterpret_cast<const float4*>(gs + i * kB32Keys + kk0);
                const float pj[4] = {pv.x, pv.y, pv.z, pv.w}, gj[4] = {gv.x, gv.y, gv.z, gv.w};
                const float* op = dor + i * (DP + 4) + d0;
                const float* qp = qr + i * (DP + 4) + d0;
#pragma unroll
                for (int e = 0; e < DC; e += 2) {
                    const float2 ov = *reinterpret_cast<const float2*>(op + e);
                    const float2 qv2 = *reinterpret_cast<const float2*>(qp + e);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        dv[j][e] = fmaf(pj[j], ov.x, dv[j][e]);
                        dv[j][e + 1] = fmaf(pj[j], ov.y, dv[j][e + 1]);
                        dk[j][e] = fmaf(gj[j], qv2.x, dk[j][e]);
                        dk[j][e + 1] = fmaf(gj[j], qv2.y, dk[j][e + 1]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int key = k0 + kk0 + j;
        if (key < Lk) {
#pragma unroll
            for (int e = 0; e < DC; ++e)
                if (d0 + e < D) {
                    kv.dk[(int64_t)key * a.dks + d0 + e] = dk[j][e];
                    kv.dv[(int64_t)key * a.dvs + d0 + e] = dv[j][e];
                }
        }
    }
}

// ----------------------------------------------------------------------------
// host side

int bset_err(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(mfa_error_buffer(), 512, fmt, ap);
    va_end(ap);
    return code;
}

typedef void (*bkernel_fn)(BArgs);

struct BwdKernels {
    bkernel_fn dsum, dkdv, dq, dkdv_sum;
    int dkdv_threads;
    int dkdv_keys = 128;  // keys per dK/dV workgroup
    int dq_rows = 128;    // query rows per dQ workgroup
};

template <int DP, bool IS_BF16>
BwdKernels bwd_kernels(bool bias) {
    BwdKernels k;
    k.dsum = mfa_bwd_dsum_kernel<IS_BF16>;
    k.dkdv_sum = mfa_bwd_dkdv_sum_kernel<IS_BF16>;
    if constexpr (DP > 64 && MFA_BWD_DKDV8) {
        k.dkdv = bias ? (bkernel_fn)mfa_bwd_dkdv8_kernel<DP, IS_BF16, true>
                      : (bkernel_fn)mfa_bwd_dkdv8_kernel<DP, IS_BF16, false>;
        k.dkdv_threads = kB8Threads;
    } else {
        k.dkdv = bias ? (bkernel_fn)mfa_bwd_dkdv_kernel<DP, IS_BF16, true>
                      : (bkernel_fn)mfa_bwd_dkdv_kernel<DP, IS_BF16, false>;
        k.dkdv_threads = kBThreads;
    }
    k.dq = bias ? (bkernel_fn)mfa_bwd_dq_kernel<DP, IS_BF16, true> : (bkernel_fn)mfa_bwd_dq_kernel<DP, IS_BF16, false>;
    return k;
}
template <bool IS_BF16>
BwdKernels bwd_select(int dp, bool bias) {
    switch (dp) {
        case 32: return bwd_kernels<32, IS_BF16>(bias);
        case 64: return bwd_kernels<64, IS_BF16>(bias);
        case 96: return bwd_kernels<96, IS_BF16>(bias);
        default: return bwd_kernels<128, IS_BF16>(bias);
    }
}

template <int DP>
BwdKernels bwd32_kernels() {
    BwdKernels k;
    k.dsum = mfa_bwd32_dsum_kernel;
    k.dkdv = mfa_bwd32_dkdv_kernel<DP>;
    k.dq = mfa_bwd32_dq_kernel<DP>;
    k.dkdv_sum = nullptr;  // (one workgroup per K/V head's keys: no partials)
    k.dkdv_threads = kBThreads;
    k.dkdv_keys = kB32Keys;
    k.dq_rows = kB32Rows;
    return k;
}
BwdKernels bwd32_select(int dp) {
    switch (dp) {
        case 32: return bwd32_kernels<32>();
        case 64: return bwd32_kernels<64>();
        case 96: return bwd32_kernels<96>();
        default: return bwd32_kernels<128>();
    }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct BPlan {
    BArgs a;
    BwdKernels k;
    int grid_dsum, grid_dkdv, grid_dq, grid_dkdv_sum;
    int64_t dsum_bytes;  // workspace: row sums first, then the dK/dV partials
    int64_t ws_bytes;
    bool empty;
};

int make_bplan(const mfa_bwd_params* bp, BPlan* plan) {
    if (!bp) return bset_err(MFA_ERR_INVALID, "mfa_bwd: params is NULL");
    const mfa_fwd_params* p = &bp->fwd;
    const int din = p->dtype_in;
    const bool f32 = din == MFA_DTYPE_F32;
    if (din != MFA_DTYPE_F16 && din != MFA_DTYPE_BF16 && !f32)
        return bset_err(MFA_ERR_UNSUPPORTED, "mfa_bwd: dtype_in %d (the backward takes bf16/fp16/fp32)", din);
    if (p->dtype_out != din)
        return bset_err(MFA_ERR_UNSUPPORTED, "mfa_bwd: o and dout must have dtype_in");
    if (bp->dtype_grad != din && bp->dtype_grad != MFA_DTYPE_F32)
        return bset_err(MFA_ERR_INVALID, "mfa_bwd: dtype_grad %d must equal dtype_in or be fp32", bp->dtype_grad);
    const int D = p->head_dim;
    if (D <= 0 || D > MFA_MAX_HEAD_DIM || D % 8 != 0)
        return bset_err(MFA_ERR_UNSUPPORTED, "mfa_bwd: head_dim %d (a multiple of 8 up to %d)", D, MFA_MAX_HEAD_DIM);
    if (p->batch < 0 || p->seqlen_q < 0 || p->seqlen_k < 0)
        return bset_err(MFA_ERR_INVALID, "mfa_bwd: negative batch/seqlen");
    if (p->heads_q <= 0 || p->heads_kv <= 0 || p->heads_q % p->heads_kv != 0)
        return bset_err(MFA_ERR_INVALID, "mfa_bwd: num_heads_kv (%d) must divide num_heads_q (%d)", p->heads_kv,
                        p->heads_q);
    if (!(p->softcap >= 0.f)) return bset_err(MFA_ERR_INVALID, "mfa_bwd: softcap must be >= 0");
    if (p->window_left < -1 || p->window_right < -1)
        return bset_err(MFA_ERR_INVALID, "mfa_bwd: window bounds must be >= -1");
    if ((p->cu_seqlens_q == nullptr) != (p->cu_seqlens_k == nullptr))
        return bset_err(MFA_ERR_INVALID, "mfa_bwd: cu_seqlens_q and cu_seqlens_k must both be set or both NULL");
    if (p->block_table) return bset_err(MFA_ERR_UNSUPPORTED, "mfa_bwd: paged K/V (block_table) has no backward");
    plan->empty = p->batch == 0 || p->seqlen_q == 0 || p->seqlen_k == 0;
    if (!plan->empty) {
        const void* ptrs[9] = {p->q, p->k, p->v, p->o, bp->dout, bp->dq, bp->dk, bp->dv, p->softmax_lse};
        for (int i = 0; i < 9; ++i)
            if (!ptrs[i]) return bset_err(MFA_ERR_INVALID, "mfa_bwd: NULL tensor pointer (softmax_lse is required)");
        for (int i = 0; i < 8; ++i)
            if (!al16(ptrs[i])) return bset_err(MFA_ERR_INVALID, "mfa_bwd: tensors must be 16-byte aligned");
        const int64_t s16[15] = {p->q_batch_stride, p->q_seq_stride, p->q_head_stride, p->k_batch_stride,
                                 p->k_seq_stride, p->k_head_stride, p->v_batch_stride, p->v_seq_stride,
                                 p->v_head_stride, p->o_batch_stride, p->o_seq_stride, p->o_head_stride,
                                 bp->do_batch_stride, bp->do_seq_stride, bp->do_head_stride};
        for (int i = 0; i < 15; ++i)
            if (s16[i] % (f32 ? 4 : 8) != 0)
                return bset_err(MFA_ERR_INVALID, "mfa_bwd: q/k/v/o/dout strides must be multiples of %d elements",
                                f32 ? 4 : 8);
        const int64_t sg[9] = {bp->dq_batch_stride, bp->dq_seq_stride, bp->dq_head_stride, bp->dk_batch_stride,
                               bp->dk_seq_stride, bp->dk_head_stride, bp->dv_batch_stride, bp->dv_seq_stride,
                               bp->dv_head_stride};
        for (int i = 0; i < 9; ++i)
            if (sg[i] % 4 != 0) return bset_err(MFA_ERR_INVALID, "mfa_bwd: dq/dk/dv strides must be multiples of 4 elements");
        if (p->alibi_slopes && !(p->alibi_batch_stride == 0 || p->alibi_batch_stride == p->heads_q))
            return bset_err(MFA_ERR_INVALID, "mfa_bwd: alibi_batch_stride must be 0 or heads_q");
        if (p->lse_batch_stride < 0 || p->lse_head_stride < 0)
            return bset_err(MFA_ERR_INVALID, "mfa_bwd: lse strides must be >= 0");
        // staged blocks (up to 128 rows: the dK/dV kernel's query steps above
        // head dim 64) are addressed with 32-bit byte offsets
        // (the fp32 kernels form 64-bit offsets)
        const int64_t rs[4] = {p->q_seq_stride, bp->do_seq_stride, p->k_seq_stride, p->v_seq_stride};
        for (int i = 0; i < 4; ++i)
            if (rs[i] < 0 || (!f32 && (127 * rs[i] + D) * 2 >= ((int64_t)1 << 31)))
                return bset_err(MFA_ERR_INVALID, "mfa_bwd: sequence strides must be >= 0 and span < 2 GiB per 128 rows");
    }
    const int dp = D <= 32 ? 32 : D <= 64 ? 64 : D <= 96 ? 96 : 128;
    const bool bias = p->softcap > 0.f || p->alibi_slopes != nullptr || !(p->scale > 0.f);
    plan->k = f32 ? bwd32_select(dp) : din == MFA_DTYPE_BF16 ? bwd_select<true>(dp, bias) : bwd_select<false>(dp, bias);

    BArgs& a = plan->a;
    memset(&a, 0, sizeof(a));
    KArgs& f = a.f;
    f.q = static_cast<const char*>(p->q);
    f.k = static_cast<const char*>(p->k);
    f.v = static_cast<const char*>(p->v);
    f.o = static_cast<char*>(p->o);
    f.qb = p->q_batch_stride; f.qs = p->q_seq_stride; f.qh = p->q_head_stride;
    f.kb = p->k_batch_stride; f.ks = p->k_seq_stride; f.kh = p->k_head_stride;
    f.vb = p->v_batch_stride; f.vs = p->v_seq_stride; f.vh = p->v_head_stride;
    f.ob = p->o_batch_stride; f.os = p->o_seq_stride; f.oh = p->o_head_stride;
    f.cu_q = p->cu_seqlens_q;
    f.cu_k = p->cu_seqlens_k;
    f.alibi = p->alibi_slopes;
    f.alibi_bstride = p->alibi_batch_stride;
    f.B = p->batch; f.Hq = p->heads_q; f.Hkv = p->heads_kv;
    f.Lq = p->seqlen_q; f.Lk = p->seqlen_k; f.D = D;
    f.scale = p->scale;
    f.scale_log2 = p->scale * kLog2e;
    f.softcap = p->softcap;
    f.softcap_k = p->softcap > 0.f ? 2.f * kLog2e / p->softcap : 0.f;
    f.softcap_sk = p->scale * f.softcap_k;
    const int64_t wmax = (int64_t)p->seqlen_q + (int64_t)p->seqlen_k + 1;
    f.wl = p->window_left < 0 ? -1 : (int32_t)(p->window_left > wmax ? wmax : p->window_left);
    f.wr = p->window_right < 0 ? -1 : (int32_t)(p->window_right > wmax ? wmax : p->window_right);
    f.causal = p->causal ? 1 : 0;
    f.lse = p->softmax_lse;
    f.lse_b = p->lse_batch_stride;
    f.lse_h = p->lse_head_stride;
    // (bounded before the int32 products below are formed)
    if ((int64_t)p->batch * p->heads_q * (p->seqlen_q > 1 ? p->seqlen_q : 1) > 0x7fffffffLL)
        return bset_err(MFA_ERR_INVALID, "mfa_bwd: problem too large");
    f.U = p->batch * p->heads_q;
    f.npages = 1;
    a.dout = static_cast<const char*>(bp->dout);
    a.dob = bp->do_batch_stride; a.dos = bp->do_seq_stride; a.doh = bp->do_head_stride;
    a.dq = static_cast<char*>(bp->dq);
    a.dqb = bp->dq_batch_stride; a.dqs = bp->dq_seq_stride; a.dqh = bp->dq_head_stride;
    a.dk = static_cast<char*>(bp->dk);
    a.dkb = bp->dk_batch_stride; a.dks = bp->dk_seq_stride; a.dkh = bp->dk_head_stride;
    a.dv = static_cast<char*>(bp->dv);
    a.dvb = bp->dv_batch_stride; a.dvs = bp->dv_seq_stride; a.dvh = bp->dv_head_stride;
    a.grad_f32 = bp->dtype_grad == MFA_DTYPE_F32 ? 1 : 0;
    a.dlse = bp->dlse;
    a.Ukv = p->batch * p->heads_kv;
    const int64_t rows = (int64_t)p->batch * p->heads_q * p->seqlen_q;
    plan->dsum_bytes = ((rows * 4 + 255) / 256) * 256;
    // Grouped-query heads: one dK/dV workgroup per query head (fp32 partials
    // summed afterwards) when that workspace stays within 2 GiB; otherwise
    // each workgroup loops over its K/V head's query heads.
    const int R = p->heads_q / p->heads_kv;
    const int64_t part = (int64_t)a.Ukv * p->seqlen_k * dp * 4;  // one group's dK (or dV) partials
    a.G = (!f32 && MFA_BWD_HEAD_SPLIT && R > 1 && 2 * R * part <= ((int64_t)2 << 30)) ? R : 1;
    if (a.G > 1 && dp > 64 && MFA_BWD_DKDV8) {
        // The eight-wavefront dK/dV kernel (one workgroup per CU) needs fewer
        // workgroups than the partials' traffic is worth: the fewest groups
        // (a power of two dividing R) that give >= 512 workgroups on dense
        // calls, 2048 on varlen calls (whose key tiles are counted at the
        // longest sequence).  Measured at D=128 causal, groups R / 2 / 1
        // (ms): B=1 L=8192 Hq=32 Hkv=8 2.15 / 2.09 / 2.07, B=2 L=4096
        // 1.27 / 1.21 / 1.18, B=4 L=2048 Hq=16 Hkv=8 non-causal 0.67 / 0.65 /
        // 0.61, B=1 L=8192 Hq=32 Hkv=4 2.15 / 2.10 / 2.9, config 4's varlen
        // batch 1.97 / 1.88 / 1.94.
        const int64_t ktiles = (p->seqlen_k + 127) / 128;
        const int64_t target = p->cu_seqlens_q ? 2048 : 512;
        int g = 1;
        while (g < R && (int64_t)a.Ukv * g * ktiles < target) g *= 2;
        if (g < R && R % g == 0) a.G = g;
    }
    a.ws_ld = dp;
    const int64_t part_bytes = a.G > 1 ? 2 * a.G * part : 0;
    plan->ws_bytes = plan->empty ? 0 : plan->dsum_bytes + part_bytes;
    const int64_t g1 = (int64_t)f.U * ((p->seqlen_q + 15) / 16);
    const int kt = plan->k.dkdv_keys, qt = plan->k.dq_rows;
    const int64_t g2 = (int64_t)a.Ukv * a.G * ((p->seqlen_k + kt - 1) / kt);
    const int64_t g3 = (int64_t)f.U * ((p->seqlen_q + qt - 1) / qt);
    if (g1 > 0x7fffffffLL || g2 > 0x7fffffffLL || g3 > 0x7fffffffLL)
        return bset_err(MFA_ERR_INVALID, "mfa_bwd: problem too large");
    plan->grid_dsum = (int)g1;
    plan->grid_dkdv = (int)g2;
    plan->grid_dq = (int)g3;
    const int64_t g4 = ((int64_t)a.Ukv * p->seqlen_k * (D / 4) + kBThreads - 1) / kBThreads;
    if (g4 > 0x7fffffffLL) return bset_err(MFA_ERR_INVALID, "mfa_bwd: problem too large");
    plan->grid_dkdv_sum = (int)g4;
    return MFA_OK;
}

}  // namespace

extern "C" {

int mfa_bwd_params_size(void) { return (int)sizeof(mfa_bwd_params); }

int mfa_bwd_supported(int32_t dtype_in, int32_t head_dim) {
    if (dtype_in != MFA_DTYPE_F16 && dtype_in != MFA_DTYPE_BF16 && dtype_in != MFA_DTYPE_F32) return 0;
    return head_dim > 0 && head_dim <= MFA_MAX_HEAD_DIM && head_dim % 8 == 0;
}

int64_t mfa_bwd_workspace_bytes(const mfa_bwd_params* params) {
    mfa_error_buffer()[0] = 0;
    BPlan plan;
    const int rc = make_bplan(params, &plan);
    if (rc != MFA_OK) return rc;
    return plan.ws_bytes;
}

int mfa_bwd(const mfa_bwd_params* params, void* workspace, int64_t workspace_bytes, void* stream) {
    mfa_error_buffer()[0] = 0;
    BPlan plan;
    const int rc = make_bplan(params, &plan);
    if (rc != MFA_OK) return rc;
    if (plan.empty) return MFA_OK;
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
        return bset_err(MFA_ERR_INVALID, "mfa_bwd: workspace must be a 256-byte aligned device pointer");
    if (workspace_bytes < plan.ws_bytes)
        return bset_err(MFA_ERR_INVALID, "mfa_bwd: workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
                        (long long)plan.ws_bytes);
    BArgs& a = plan.a;
    a.dsum = static_cast<float*>(workspace);
    if (a.G > 1) {
        a.ws_dk = reinterpret_cast<float*>(static_cast<char*>(workspace) + plan.dsum_bytes);
        a.ws_dv = a.ws_dk + (int64_t)a.G * a.Ukv * params->fwd.seqlen_k * a.ws_ld;
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    a.T = (params->fwd.seqlen_q + 15) / 16;
    hipLaunchKernelGGL(plan.k.dsum, dim3(plan.grid_dsum), dim3(kBThreads), 0, st, a);
    a.T = (params->fwd.seqlen_k + plan.k.dkdv_keys - 1) / plan.k.dkdv_keys;
    hipLaunchKernelGGL(plan.k.dkdv, dim3(plan.grid_dkdv), dim3(plan.k.dkdv_threads), 0, st, a);
    if (a.G > 1) hipLaunchKernelGGL(plan.k.dkdv_sum, dim3(plan.grid_dkdv_sum), dim3(kBThreads), 0, st, a);
    a.T = (params->fwd.seqlen_q + plan.k.dq_rows - 1) / plan.k.dq_rows;
    hipLaunchKernelGGL(plan.k.dq, dim3(plan.grid_dq), dim3(kBThreads), 0, st, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return bset_err(MFA_ERR_LAUNCH, "mfa_bwd: launch failed: %s", hipGetErrorString(e));
    return MFA_OK;
}

}  // extern "C"
