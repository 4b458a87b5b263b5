// mfa_fwd.hip -- MI355X (gfx950 / CDNA4) flash-attention forward kernels and
// the C ABI declared in include/mfa.h.
//
// Reference semantics: metal_flash_attn/_kernel.py:32-87 (the scalar v0 kernel
// states the mask/bias/online-softmax math most plainly) and :1165-1208 (the
// chunked fp32 torch path, whose results these kernels must reproduce).
//
// Kernels: mfa_fwd16_kernel (bf16/fp16, 4 wavefronts; its EXACT
// instantiation serves single query rows with two-term probabilities),
// mfa_fwd16_pp_kernel (bf16/fp16, 8 wavefronts on a ping-pong schedule: the
// two wavefronts of a SIMD alternate MFMA and softmax phases),
// mfa_fwd16_tk_kernel (at most 32 keys per sequence), mfa_fwd32_kernel
// (fp32) and mfa_combine_kernel (split-KV merge).  Grouped-query calls pack
// the query heads of one K/V head into a tile (each wavefront still holds
// 32 aligned positions of one head).  Shared design:
//  * The score tile is computed TRANSPOSED, S^T = K * Q^T, with
//    v_mfma_f32_32x32x16_{bf16,f16} (fp32 inputs: v_mfma_f32_32x32x2_f32).
//    In the 32x32 MFMA accumulator layout lane l holds column l%32, so every
//    lane owns exactly one query row: max/sum/rescale are lane-local and the
//    only cross-lane step per K/V block is one v_permlane32_swap to merge the
//    two half-waves that share a query.
//  * O is accumulated transposed as well, O^T = V^T * P^T, whose accumulator
//    again gives each lane one query, so the online-softmax rescale of O is a
//    lane-local multiply.  P^T is fed to the MFMA straight from the S^T
//    accumulator registers (converted to bf16/f16 in registers); it never
//    touches LDS.  The k-slot order of that MFMA follows the accumulator
//    row order; V stays row-major in LDS and its transposed operand is read
//    with ds_read_b64_tr_b16 (gfx950 LDS transpose loads).
//  * Q is staged through LDS once (coalesced global reads) and then lives in
//    registers as the MFMA B operand.  K and V stream through two LDS buffers:
//    the global loads of block j+1 are issued before the MFMAs of block j and
//    written to the other buffer after them, one barrier per block.
//  * Keys outside [lo(q), hi(q)] (bottom-right causal, sliding window, the
//    sequence end) are skipped a whole block at a time where a block is
//    entirely outside the range of every query of the workgroup, masked
//    element-wise only on the boundary blocks of each wavefront, and
//    untouched elsewhere.
//  * O and l are rescaled only in blocks where some row's max grew by more
//    than a factor 2 (a wave-uniform branch); the reference max then becomes
//    every row's exact max, so probabilities stay <= 2 and the row's largest
//    weight is within one binade of 1.0 when P is rounded to 16 bits.
//  * O leaves through non-temporal stores (row-contiguous 16-byte pieces,
//    staged through LDS, in the 16-bit kernels): it is never read back here.
//  * Where the number of K/V head groups is a multiple of 8, all tiles of one
//    K/V head run on one XCD, so its K/V stays in that XCD's L2: one
//    (sequence, q head) after another when tiles cost the same, heaviest
//    tiles of every unit first under causal masks and windows (head-packed
//    varlen tiles keep the unit order, see decode_tile and make_plan).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <type_traits>
#include <utility>

#include "mfa.h"
#include "mfa_common.h"

namespace {


constexpr int kWaves = 4;
// wavefronts per SIMD the 16-bit kernels are register-budgeted for
#ifndef MFA_WAVES_PER_EU
#define MFA_WAVES_PER_EU 2
#endif
// exp2-domain growth of a row max below which the wave keeps its previous
// reference max (0: move whenever any row's max grows)
#ifndef MFA_RESCALE_TAU
#define MFA_RESCALE_TAU 1
#endif
// padding (elements) of the row-major V tile in LDS
#ifndef MFA_V_PAD
#define MFA_V_PAD 32
#endif
// issue the next blocks' K/V staging between the last PV MFMAs
#ifndef MFA_STAGE_IN_PV
#define MFA_STAGE_IN_PV 1
#endif
// stage the next blocks without branches in the pipelined path
#ifndef MFA_BRANCHFREE_STAGE
#define MFA_BRANCHFREE_STAGE 1
#endif
// raise the wave priority around the MFMA-only stretches of a pipelined block
#ifndef MFA_SETPRIO
#define MFA_SETPRIO 0
#endif
// ... and around the QK^T and PV MFMAs of a sequential block
#ifndef MFA_SIMPLE_PRIO
#define MFA_SIMPLE_PRIO 1
#endif
// fragments read ahead of their MFMAs in the ping-pong kernel's MFMA phase
#ifndef MFA_PP_AHEAD
#define MFA_PP_AHEAD 2
#endif
// the same for one query block per wavefront (one MFMA per fragment), at
// head dims up to 64 and above
#ifndef MFA_PP_AHEAD1
#define MFA_PP_AHEAD1 4
#endif
#ifndef MFA_PP_AHEAD1W
#define MFA_PP_AHEAD1W 2
#endif
// raise the wave priority during the MFMA phase of the ping-pong kernel
#ifndef MFA_PP_PRIO
#define MFA_PP_PRIO 1
#endif
// ping-pong kernel with four wavefronts per SIMD (512-row tiles of one 32-row
// query block per wavefront) at head dims up to 64, and its operand read-ahead
#ifndef MFA_PP_NW16
#define MFA_PP_NW16 0
#endif
#ifndef MFA_PP_AHEAD16
#define MFA_PP_AHEAD16 1
#endif
// ping-pong kernel: group 1 issues its K/V loads in its MFMA phase
#ifndef MFA_PP_DMA_A
#define MFA_PP_DMA_A 1
#endif
// ping-pong kernel: the row sums of a block's rounded probabilities are
// issued at the start of the next MFMA phase (dot2 instructions wait while
// the other wavefront of the SIMD issues MFMAs, which it does not at that
// point) ...
#ifndef MFA_PP_SUM_IN_A
#define MFA_PP_SUM_IN_A 1
#endif
// ... or, with that off, after all of the block's probabilities, late in the
// softmax phase, when the partner wavefront's MFMAs are mostly done
#ifndef MFA_PP_LATE_SUM
#define MFA_PP_LATE_SUM 1
#endif
// software-pipelined unmasked blocks (QB >= 2)
#ifndef MFA_PIPELINE
#define MFA_PIPELINE 1
#endif
// head dims above 64 with ALiBi: walk the key blocks from the last to the first
#ifndef MFA_ALIBI_REVERSE
#define MFA_ALIBI_REVERSE 1
#endif
constexpr int kThreads = kWaves * 64;

// ----------------------------------------------------------------------------
// Online softmax on S^T accumulators (shared by the 16-bit and fp32 kernels,
// which use the same 32x32 accumulator layout).
//
// For one 32-query block, s[kb][r] is the raw score of query (lane%32) and
// key j + 32*kb + 4*(lane/32) + acc_row(r).  The softmax of one K/V block is
//   transform  : scale / soft-cap / ALiBi (BIAS) and masking (MASKED)
//   row max    : over the lane's keys, merged across the two half-waves
//   update     : new running max, rescale factor alpha for O and l
//   probs      : p = exp2(s*c - mu), rounded to 16 bits for the PV MFMA,
//                l += sum(p) (of the rounded values)

// per-lane state of the query row a lane owns
struct RowState {
    int center;  // bottom-right diagonal: q + Lk - Lq
    int lo, hi;  // valid key interval [lo, hi]
    float slope; // ALiBi slope (0 without ALiBi)
    float m;     // running max (raw-score units without BIAS, natural-log units with)
    float mu;    // exponent offset m*c of the probabilities (0 while m = -inf)
    float thr;   // m + tau/c: a larger block max moves the reference
    float l;     // running row sum (this half-wave's keys)
};

// Smallest ALiBi distance |center - j| over the row's valid keys [lo, hi].
__device__ __forceinline__ int row_dmin(const RowState& rs) {
    return max(0, max(rs.lo - rs.center, rs.center - rs.hi));
}

// PRECISE (the fp32 kernel): x = s*scale, softcap*tanh(x/softcap) with the
// precise tanh, then ALiBi as -slope*(|d| - dmin), dmin = row_dmin (the
// softmax is unchanged by a per-row constant; the lse store adds
// -slope*dmin back).  A row hundreds of keys from every key then keeps its
// scores near zero instead of near -slope*|d| (~ -10^2, where fp32 spacing
// is ~1e-5).  The 16-bit kernels keep the fused forms.
template <int NKB, bool BIAS, bool MASKED, bool PRECISE = false>
__device__ __forceinline__ void qb_transform(const KArgs& a, f32x16_t (&s)[NKB], const RowState& rs, int j,
                                             int half) {
    if constexpr (BIAS && PRECISE) {
        const float dmin = (float)row_dmin(rs);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            const float cf = (float)(rs.center - (j + 32 * kb + 4 * half));
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float x = s[kb][r] * a.scale;
                if (a.softcap > 0.f) x = a.softcap * precise_tanh(__fdiv_rn(x, a.softcap));
                if (a.alibi) x = fmaf(-rs.slope, fabsf(cf - (float)acc_row(r)) - dmin, x);
                s[kb][r] = x;
            }
        }
    } else if constexpr (BIAS) {
        // natural-log units: x = scale*s, soft-cap, ALiBi (_kernel.py:75-77)
        if (a.softcap > 0.f) {
            // c * tanh(x / c) = c - 2c / (exp(2x/c) + 1), the scale folded
            // into the exponent's constant (x itself is not needed)
            const float c2 = -2.f * a.softcap;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float e = fast_exp2(s[kb][r] * a.softcap_sk);
                    s[kb][r] = fmaf(c2, __builtin_amdgcn_rcpf(e + 1.f), a.softcap);
                }
        } else {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) s[kb][r] *= a.scale;
        }
        if (a.alibi) {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                const float cf = (float)(rs.center - (j + 32 * kb + 4 * half));
#pragma unroll
                for (int r = 0; r < 16; ++r) s[kb][r] = fmaf(-rs.slope, fabsf(cf - (float)acc_row(r)), s[kb][r]);
            }
        }
    }
    if constexpr (MASKED) {
        // (the pinned copy keeps the compiler from hoisting the 32 key
        // indices out of the masked path into every block)
        int jm = j;
        asm volatile("" : "+v"(jm));
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            const int kbase = jm + 32 * kb + 4 * half;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kbase + acc_row(r);
                s[kb][r] = ((key >= rs.lo) & (key <= rs.hi)) ? s[kb][r] : -INFINITY;
            }
        }
    }
}

// (two independent max chains, so consecutive instructions do not wait on
// each other's results)
template <int NKB>
__device__ __forceinline__ float qb_max(const f32x16_t (&s)[NKB]) {
    float m0 = s[0][0], m1 = s[0][1];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            if (kb == 0 && r == 0) continue;
            m0 = fmax_nn(m0, s[kb][r]);
            m1 = fmax_nn(m1, s[kb][r + 1]);
        }
    return max_halves(fmax_nn(m0, m1));
}

// Running-max update from the block max mx.  The reference max of the wave
// moves (to every row's exact max) only when some row's block max exceeds its
// threshold thr = m + tau/c, i.e. grew by more than tau (MFA_RESCALE_TAU) in
// the exp2 domain; otherwise probabilities are taken against the previous
// reference, so p <= 2^tau.  O and l always use the same reference, so the
// final O/l is unaffected.  The exponent offset mu = m*c and thr change only
// on a move, so a block that moves no row costs one compare per row.  Rows
// with no valid key so far keep m = thr = -inf and mu = 0, so masked scores
// give p = 0.  With tau = 0 a row whose max did not grow gets
// alpha = exp2(0) = 1 exactly, so each row's arithmetic is independent of
// the other rows of its wave.
__device__ __forceinline__ void row_reset(RowState& rs) {
    rs.m = -INFINITY;
    rs.thr = -INFINITY;
    rs.mu = 0.f;
    rs.l = 0.f;
}
// Returns true when the reference moved (wave-uniform); m_old keeps the
// previous running max, for the rescale factor move_alpha(m_old, m, c) the
// caller applies to O and l only then.  tau_c = tau / c.
__device__ __forceinline__ bool qb_move(RowState& rs, float mx, float c, float tau_c, float& m_old) {
    m_old = rs.m;
    const bool moved = __any(mx > rs.thr);
    if (moved) {
        rs.m = fmax_nn(rs.m, mx);
        rs.mu = rs.m == -INFINITY ? 0.f : rs.m * c;
        rs.thr = rs.m + tau_c;
    }
    return moved;
}
__device__ __forceinline__ float move_alpha(float m_old, float m_new, float c) {
    return m_new == -INFINITY ? 1.f : fast_exp2((m_old - m_new) * c);
}
// qb_move with the rescale of l; alpha is the factor for O when it returns true
__device__ __forceinline__ bool qb_update(RowState& rs, float mx, float c, float tau_c, float& alpha) {
    float m_old;
    alpha = 1.f;
    const bool moved = qb_move(rs, mx, c, tau_c, m_old);
    if (moved) {
        alpha = move_alpha(m_old, rs.m, c);
        rs.l *= alpha;
    }
    return moved;
}

template <int DB>
__device__ __forceinline__ void scale_rows(f32x16_t (&o)[DB], float alpha) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2_t;

// Two probabilities rounded to 16 bits, packed, and added (as rounded) to acc:
// the row sum l is the sum of exactly the weights the PV MFMA consumes.
template <bool IS_BF16>
__device__ __forceinline__ uint32_t pack_and_sum(float p0, float p1, float& acc) {
    if constexpr (IS_BF16) {
        const bf16x2_t pk = {(__bf16)p0, (__bf16)p1};
        const bf16x2_t one = {(__bf16)1.f, (__bf16)1.f};
        acc = __builtin_amdgcn_fdot2_f32_bf16(pk, one, acc, false);
        return __builtin_bit_cast(uint32_t, pk);
    } else {
        const f16x2_t pk = {(_Float16)p0, (_Float16)p1};
        const f16x2_t one = {(_Float16)1.f, (_Float16)1.f};
        acc = __builtin_amdgcn_fdot2(pk, one, acc, false);
        return __builtin_bit_cast(uint32_t, pk);
    }
}

// P^T B operands straight from the accumulators: pw[kb][st] holds
// accumulator registers 8*st..8*st+7 of key block kb.
// (the block's row sum starts from zero in two independent chains and is
// added to l at the end, so the sums do not wait for l's rescale)
template <int NKB, bool IS_BF16>
__device__ __forceinline__ void qb_probs16(const f32x16_t (&s)[NKB], u32x4_t (&pw)[NKB][2], float& l, float mu,
                                           float c) {
    float acc[2] = {0.f, 0.f};  // two independent sum chains
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float p0 = fast_exp2(fmaf(s[kb][8 * st + 2 * w], c, -mu));
                const float p1 = fast_exp2(fmaf(s[kb][8 * st + 2 * w + 1], c, -mu));
                pw[kb][st][w] = pack_and_sum<IS_BF16>(p0, p1, acc[w & 1]);
            }
    l += acc[0] + acc[1];
}

// qb_probs16 in two passes: the rounded probabilities, then (called later)
// their row sum.  The same values are summed in the same order, so l is
// bit-identical to qb_probs16's.
template <int NKB, bool IS_BF16>
__device__ __forceinline__ void qb_probs16_only(const f32x16_t (&s)[NKB], u32x4_t (&pw)[NKB][2], float mu,
                                                float c) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float p0 = fast_exp2(fmaf(s[kb][8 * st + 2 * w], c, -mu));
                const float p1 = fast_exp2(fmaf(s[kb][8 * st + 2 * w + 1], c, -mu));
                if constexpr (IS_BF16) {
                    const bf16x2_t pk = {(__bf16)p0, (__bf16)p1};
                    pw[kb][st][w] = __builtin_bit_cast(uint32_t, pk);
                } else {
                    const f16x2_t pk = {(_Float16)p0, (_Float16)p1};
                    pw[kb][st][w] = __builtin_bit_cast(uint32_t, pk);
                }
            }
}
template <int NKB, bool IS_BF16>
__device__ __forceinline__ float qb_sum16(const u32x4_t (&pw)[NKB][2]) {
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                // (a plain copy first: a bit cast straight from a vector element
                // reads element 0 with this compiler)
                const uint32_t x = pw[kb][st][w];
                if constexpr (IS_BF16) {
                    const bf16x2_t one = {(__bf16)1.f, (__bf16)1.f};
                    acc[w & 1] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x), one, acc[w & 1], false);
                } else {
                    const f16x2_t one = {(_Float16)1.f, (_Float16)1.f};
                    acc[w & 1] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x), one, acc[w & 1], false);
                }
            }
    return acc[0] + acc[1];
}

// Two-term 16-bit probabilities, for rows whose O averages so many
// near-equal weights that one 16-bit rounding of each weight is visible
// against max|O| (single-row sequences and packed grouped-query decode rows):
// hi = round16(p) and lo = round16(p - hi) (the difference is exact in fp32).
// The PV MFMA consumes both against the same V fragment, so the weights carry
// about 16 mantissa bits instead of 8 (bf16) or 11 (fp16).  The row sum adds
// the fp32 weights themselves (two chains, acc[0] and acc[1]), which hi + lo
// reproduce to 2^-17 relative (plain adds: two dot2 per pair measured 1.2%
// slower on single-row decode).
// One group: the 8 weights of accumulator registers 8*st..8*st+7.
template <bool IS_BF16>
__device__ __forceinline__ void probs16x2_group(const f32x16_t& s, int st, u32x4_t& ph, u32x4_t& pl,
                                                float (&acc)[2], float mu, float c) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float p0 = fast_exp2(fmaf(s[8 * st + 2 * w], c, -mu));
        const float p1 = fast_exp2(fmaf(s[8 * st + 2 * w + 1], c, -mu));
        float h0, h1;
        if constexpr (IS_BF16) {
            const bf16x2_t hk = {(__bf16)p0, (__bf16)p1};
            const uint32_t h = __builtin_bit_cast(uint32_t, hk);
            h0 = __builtin_bit_cast(float, h << 16);
            h1 = __builtin_bit_cast(float, h & 0xffff0000u);
            const bf16x2_t lk = {(__bf16)(p0 - h0), (__bf16)(p1 - h1)};
            ph[w] = h;
            pl[w] = __builtin_bit_cast(uint32_t, lk);
        } else {
            const f16x2_t hk = {(_Float16)p0, (_Float16)p1};
            h0 = (float)hk[0];
            h1 = (float)hk[1];
            const f16x2_t lk = {(_Float16)(p0 - h0), (_Float16)(p1 - h1)};
            ph[w] = __builtin_bit_cast(uint32_t, hk);
            pl[w] = __builtin_bit_cast(uint32_t, lk);
        }
        acc[w & 1] += p0 + p1;
    }
}

template <int NKB>
__device__ __forceinline__ void qb_probs32(f32x16_t (&s)[NKB], float& l, float mu, float c) {
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = fast_exp2(fmaf(s[kb][r], c, -mu));
            s[kb][r] = p;
            acc[r & 1] += p;
        }
    l += acc[0] + acc[1];
}

// Normalise and store O^T accumulators: lane (half, q) holds
// d = 32*db + 8*g + 4*half + {0..3} for g = 0..3.  With an lse output the
// row's natural-log log-sum-exp (mu + log2 l) * ln 2 is stored too (the
// probabilities were exp2(x*c - mu), l their sum), -inf for a row with no
// valid key.
constexpr float kLn2 = 0.6931471805599453f;
// lsum[qb]: the row sum of query block qb for this lane's query (both halves)
template <int QB, int DB, bool IS_BF16>
__device__ __forceinline__ void store_out_l(const KArgs& a, const SeqView& sv, f32x16_t (&o)[QB][DB],
                                            const RowState (&rs)[QB], const float (&lsum)[QB], int qrow0, int lane,
                                            float c) {
    const int l32 = lane & 31, half = lane >> 5;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const float l = lsum[qb];
        const float inv = l > 0.f ? 1.f / l : 0.f;  // fully masked rows -> 0 (_kernel.py:85)
        const int qrow = qrow0 + 32 * qb + l32;
        if (qrow >= sv.Lq) continue;
        if (sv.lse && half == 0) {
            const float mu = rs[qb].mu;
            sv.lse[qrow] = l > 0.f ? (mu + __builtin_amdgcn_logf(l)) * kLn2 : -INFINITY;
        }
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * db + 8 * g + 4 * half;
                if (d >= a.D) continue;
                const float v0 = o[qb][db][4 * g + 0] * inv, v1 = o[qb][db][4 * g + 1] * inv;
                const float v2 = o[qb][db][4 * g + 2] * inv, v3 = o[qb][db][4 * g + 3] * inv;
                if (a.out_f32) {
                    float* dst = reinterpret_cast<float*>(sv.o) + (int64_t)qrow * a.os + d;
                    typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4v_t;
                    store_stream(reinterpret_cast<f32x4v_t*>(dst), f32x4v_t{v0, v1, v2, v3});
                } else if constexpr (IS_BF16) {
                    typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
                    bf16x4_t w = {(__bf16)v0, (__bf16)v1, (__bf16)v2, (__bf16)v3};
                    store_stream(reinterpret_cast<bf16x4_t*>(reinterpret_cast<__bf16*>(sv.o) + (int64_t)qrow * a.os + d), w);
                } else {
                    typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4_t;
                    f16x4_t w = {(_Float16)v0, (_Float16)v1, (_Float16)v2, (_Float16)v3};
                    store_stream(reinterpret_cast<f16x4_t*>(reinterpret_cast<_Float16*>(sv.o) + (int64_t)qrow * a.os + d), w);
                }
            }
    }
}
// row sums kept per half-wave in rs[qb].l
template <int QB, int DB, bool IS_BF16>
__device__ __forceinline__ void store_out(const KArgs& a, const SeqView& sv, f32x16_t (&o)[QB][DB],
                                          const RowState (&rs)[QB], int qrow0, int lane, float c) {
    float lsum[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) lsum[qb] = sum_halves(rs[qb].l);
    store_out_l<QB, DB, IS_BF16>(a, sv, o, rs, lsum, qrow0, lane, c);
}

// store_out with the 16-bit rows routed through this wavefront's LDS block
// `ls` (32*QB rows of ST elements), so that the global stores are
// row-contiguous -- 16 lanes per 256-byte row -- instead of 32 rows in
// 8-byte pieces per instruction.  The same values as store_out; the fp32
// parity output keeps the direct store.
#ifndef MFA_LDS_OSTORE
#define MFA_LDS_OSTORE 1
#endif
template <int QB, int DB, bool IS_BF16, int ST>
__device__ __forceinline__ void store_out_rows(const KArgs& a, const SeqView& sv, f32x16_t (&o)[QB][DB],
                                               const RowState (&rs)[QB], int qrow0, int lane, float c,
                                               uint16_t* ls) {
    float lsum[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) lsum[qb] = sum_halves(rs[qb].l);
    if (!MFA_LDS_OSTORE || a.out_f32) {
        store_out_l<QB, DB, IS_BF16>(a, sv, o, rs, lsum, qrow0, lane, c);
        return;
    }
    // (a fresh copy of the lane id: addresses derived from it are not shared
    // with the main loop's, which would keep them live across the loop)
    asm volatile("" : "+v"(lane));
    const int l32 = lane & 31, half = lane >> 5;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const float l = lsum[qb];
        const float inv = l > 0.f ? 1.f / l : 0.f;  // fully masked rows -> 0 (_kernel.py:85)
        const int qrow = qrow0 + 32 * qb + l32;
        if (sv.lse && half == 0 && qrow < sv.Lq)
            sv.lse[qrow] = l > 0.f ? (rs[qb].mu + __builtin_amdgcn_logf(l)) * kLn2 : -INFINITY;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float v0 = o[qb][db][4 * g] * inv, v1 = o[qb][db][4 * g + 1] * inv;
                const float v2 = o[qb][db][4 * g + 2] * inv, v3 = o[qb][db][4 * g + 3] * inv;
                u32x2_t w;
                if constexpr (IS_BF16) {
                    typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
                    w = __builtin_bit_cast(u32x2_t, bf16x4_t{(__bf16)v0, (__bf16)v1, (__bf16)v2, (__bf16)v3});
                } else {
                    typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4_t;
                    w = __builtin_bit_cast(u32x2_t, f16x4_t{(_Float16)v0, (_Float16)v1, (_Float16)v2, (_Float16)v3});
                }
                *reinterpret_cast<u32x2_t*>(ls + (32 * qb + l32) * ST + 32 * db + 8 * g + 4 * half) = w;
            }
    }
    constexpr int CPR = DB * 4;                 // 16-byte chunks per row
    constexpr int NCH = 32 * QB * CPR / 64;     // per lane
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int ch = lane + 64 * i, r = ch / CPR, col = (ch % CPR) * 8;
        const u32x4_t w = *reinterpret_cast<const u32x4_t*>(ls + r * ST + col);
        const int qrow = qrow0 + r;
        if (qrow < sv.Lq && col < a.D) store_stream(reinterpret_cast<u32x4_t*>(sv.o + ((int64_t)qrow * a.os + col) * 2), w);
    }
}

// Split-KV partial of one chunk: O normalised by the chunk's own row sum and
// the chunk's log2-sum-exp lse = mu + log2(l) (probabilities were
// exp2(x - mu)); a row with no valid key in the chunk gets lse = -inf, O = 0.
template <int QB, int DB>
__device__ __forceinline__ void store_partial(const KArgs& a, int Lq, int unit, int split, f32x16_t (&o)[QB][DB],
                                              const RowState (&rs)[QB], float c, int qrow0, int lane) {
    const int l32 = lane & 31, half = lane >> 5;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const float l = sum_halves(rs[qb].l);
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const int qrow = qrow0 + 32 * qb + l32;
        if (qrow >= Lq) continue;
        const int64_t row = ((int64_t)split * a.U + unit) * a.Lq + qrow;
        if (half == 0) {
            const float mu = rs[qb].mu;
            a.ws_lse[row] = l > 0.f ? mu + __builtin_amdgcn_logf(l) : -INFINITY;
        }
        float* dst = a.ws_o + row * a.ws_ld;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * db + 8 * g + 4 * half;
                if (d >= a.D) continue;
                *reinterpret_cast<float4*>(dst + d) =
                    make_float4(o[qb][db][4 * g] * inv, o[qb][db][4 * g + 1] * inv, o[qb][db][4 * g + 2] * inv,
                                o[qb][db][4 * g + 3] * inv);
            }
    }
}

// Merge of the split-KV partials, one wavefront per query row (and the
// row's lse when requested: M + log2(sum_s w_s), in natural-log units).  A sequence
// uses ceil(Lk / split_keys) chunks (one when it has no key); O =
// sum_s w_s O_s / sum_s w_s with w_s = 2^(lse_s - M), M = max_s lse_s, and 0
// when no chunk has a valid key (a fully masked row, _kernel.py:85-86).  The
// lanes read the chunks' lse in parallel (max and weight sum reduced across
// the wavefront, weights kept in LDS), then each lane sums its two head-dim
// elements over the chunks in chunk order with independent loads.  With one
// chunk the weight is exactly 1 and O is the chunk's O unchanged.
constexpr int kMaxSplits = 1024;
template <bool IS_BF16>
__global__ void __launch_bounds__(64) mfa_combine_kernel(KArgs a) {
    __shared__ float wsh[kMaxSplits];
    const int lane = threadIdx.x;
    const int64_t r = blockIdx.x;  // row (unit, query row)
    const int unit = (int)(r / a.Lq), qrow = (int)(r % a.Lq);
    const int b = unit / a.Hq, hq = unit - b * a.Hq;
    const SeqView sv = seq_view<2>(a, b, hq);
    if (qrow >= sv.Lq) return;
    const int ns = min(a.nsplit, max(1, (sv.Lk + a.split_keys - 1) / a.split_keys));
    const int64_t stride = (int64_t)a.U * a.Lq;
    float m = -INFINITY;
    for (int sp = lane; sp < ns; sp += 64) m = fmaxf(m, a.ws_lse[sp * stride + r]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float wsum = 0.f;
    for (int sp = lane; sp < ns; sp += 64) {
        const float lse = a.ws_lse[sp * stride + r];
        const float w = m == -INFINITY || lse == -INFINITY ? 0.f : fast_exp2(lse - m);
        wsh[sp] = w;
        wsum += w;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) wsum += __shfl_xor(wsum, o);
    if (sv.lse && lane == 0)  // natural-log lse of the merged row
        sv.lse[qrow] = m == -INFINITY ? -INFINITY : (m + __builtin_amdgcn_logf(wsum)) * kLn2;
    __syncthreads();
    const int d = 2 * lane;
    if (d >= a.D) return;
    float acc0 = 0.f, acc1 = 0.f;
    if (m != -INFINITY) {
        const float* src = a.ws_o + r * a.ws_ld + d;
#pragma unroll 8
        for (int sp = 0; sp < ns; ++sp) {
            const float2 x = *reinterpret_cast<const float2*>(src + sp * stride * a.ws_ld);
            acc0 = fmaf(wsh[sp], x.x, acc0);
            acc1 = fmaf(wsh[sp], x.y, acc1);
        }
        acc0 /= wsum;
        acc1 /= wsum;
    }
    if (a.out_f32) {
        typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2v_t;
        store_stream(reinterpret_cast<f32x2v_t*>(reinterpret_cast<float*>(sv.o) + (int64_t)qrow * a.os + d),
                     f32x2v_t{acc0, acc1});
    } else if constexpr (IS_BF16) {
        const bf16x2_t w = {(__bf16)acc0, (__bf16)acc1};
        store_stream(reinterpret_cast<bf16x2_t*>(reinterpret_cast<__bf16*>(sv.o) + (int64_t)qrow * a.os + d), w);
    } else {
        const f16x2_t w = {(_Float16)acc0, (_Float16)acc1};
        store_stream(reinterpret_cast<f16x2_t*>(reinterpret_cast<_Float16*>(sv.o) + (int64_t)qrow * a.os + d), w);
    }
}

// ----------------------------------------------------------------------------
// 16-bit (bf16 / fp16) kernel.
//   DP  : head dim padded to a multiple of 32 (32, 64, 96, 128)
//   QB  : 32-query column blocks per wavefront (workgroup rows = 4*32*QB)
//   NKB : 32-key row blocks per K/V block (keys per block = 32*NKB)
//   EXACT: the exact-row instantiation (block_exact below): the kernel of
//          single-row sequences and packed grouped-query decode rows.  It is
//          a separate kernel, not a path of the others: a second block path
//          inside their key loop made the register allocator spill in it.
// With QB >= 2, unmasked blocks run software-pipelined: the QK^T MFMAs of
// query block qb+1 and the PV MFMAs of query block qb-1 are interleaved with
// the softmax VALU work of query block qb, so the matrix cores and the
// vector ALU run concurrently within one wavefront.
template <int DP, int QB, int NKB, bool IS_BF16, bool BIAS, bool PAGED, bool EXACT>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(MFA_WAVES_PER_EU)))
mfa_fwd16_kernel(KArgs a) {
    constexpr int BM = kWaves * QB * 32;
    constexpr int BN = NKB * 32;
    constexpr int DS = DP / 16;  // QK^T k-steps
    constexpr int DB = DP / 32;  // O^T row blocks
    constexpr int KST = DP + 8;  // K / Q LDS row stride (elements): +16 B against bank conflicts
    // V row stride: 2*VST = 64 (mod 256) bytes, so the 4 rows x 64 bytes that a
    // half-wave's transpose read touches fall on disjoint banks
    constexpr int VST = DP + MFA_V_PAD;
    constexpr int K_ELEMS = BN * KST;
    constexpr int V_ELEMS = BN * VST;
    constexpr int KV_ELEMS = 2 * (K_ELEMS + V_ELEMS);
    constexpr int Q_ELEMS = BM * KST;
    // The exact-row kernel's LDS is sized (at least 60 KB) so that two
    // workgroups share a CU, as with the other kernels' tiles: its decode
    // workgroups are HBM-streaming, and three per CU at head dim 64 (what
    // its registers and 43 KB of K/V stages would allow) measured 18% slower
    // than two (B=64 H=16 Lk=4096 D=64 single rows: 0.238 against 0.201 ms).
    constexpr int SMEM_KV = KV_ELEMS > Q_ELEMS ? KV_ELEMS : Q_ELEMS;
    constexpr int SMEM = (EXACT && SMEM_KV < 30000) ? 30000 : SMEM_KV;
    constexpr int CPR = DP / 8;                                 // 16-byte chunks per row
    constexpr int KCH = (BN * CPR + kThreads - 1) / kThreads;  // chunks per thread per tile
    typedef typename std::conditional<IS_BF16, bf16x8_t, f16x8_t>::type op_t;

    __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM];

    int b, hq, tile;
    if (!decode_tile(a, blockIdx.x, b, hq, tile)) return;
    int split = 0;
    if (a.nsplit > 1) {
        split = tile % a.nsplit;
        tile /= a.nsplit;
    }
    const SeqView sv = seq_view<2>(a, b, hq);
    // Head-packed tiles (a.hpack = R > 1, grouped-query calls): the tile
    // holds PM positions of each of the R query heads of one K/V head,
    // head-major (tile row = head * PM + position); wave w takes head
    // w / (kWaves / R) at position block w % (kWaves / R), so it still holds
    // QB * 32 aligned positions of one head and its rows' arithmetic equals
    // the unpacked tile's.
    const int hpk = EXACT ? 1 : a.hpack;
    const int PM = BM / hpk;  // positions per tile
    const int q0 = tile * PM;
    if (q0 >= sv.Lq) return;
    // a varlen call mixing single-row sequences with longer ones: the
    // exact-row kernel's launch takes the single-row ones, this one the rest
    if (a.single_rows != 0 && (sv.Lq == 1) != EXACT) return;
    // split-KV: this sequence's chunks (one when it has no key)
    if (a.nsplit > 1 && split >= max(1, (sv.Lk + a.split_keys - 1) / a.split_keys)) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int Lq = sv.Lq, Lk = sv.Lk, D = a.D;
    const int dq = Lk - Lq;

    const int wph = kWaves / hpk;                      // waves per head
    const int hl = wave / wph;                         // this wave's head inside the tile
    const int wq0 = q0 + (wave - hl * wph) * QB * 32;  // first query row of this wavefront
    op_t qf[QB][DS];                                   // Q as MFMA B operands (filled below)


    // ---- per-lane query state
    RowState rs[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        rs[qb].center = wq0 + 32 * qb + l32 + dq;
        rs[qb].lo = key_lo(a, rs[qb].center);
        rs[qb].hi = key_hi(a, rs[qb].center, Lk);
        rs[qb].slope = a.alibi ? a.alibi[b * a.alibi_bstride + hq * hpk + hl] : 0.f;
        row_reset(rs[qb]);
    }
    f32x16_t o[QB][DB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[qb][db][r] = 0.f;
    const float c = BIAS ? kLog2e : a.scale_log2;
    // Exact rows (this instantiation's: single-row sequences and packed
    // grouped-query decode rows) take per-row rescales -- their results do not
    // depend on which rows share a wave, so packed heads equal unpacked ones
    // bit for bit -- and two-term probabilities (block_exact): a single row
    // averaging thousands of near-equal weights has a small max|O|, against
    // which one 16-bit rounding of every weight is visible.
    const float tau = (EXACT || Lq == 1 || a.decode_pack) ? 0.f : (float)MFA_RESCALE_TAU;
    const float tau_c = tau / c;

    // ---- key range of the workgroup and of this wavefront
    const int qlast = min(q0 + PM, Lq) - 1;
    const int klo = key_lo(a, q0 + dq);
    const int khi = key_hi(a, qlast + dq, Lk);
    int jbeg = (klo / BN) * BN;
    int nblk = khi >= klo ? (khi - jbeg) / BN + 1 : 0;
    int kend = Lk;  // loads read zero from key kend on
    if (a.nsplit > 1) {
        // split-KV: the blocks of chunk `split` (chunks are whole blocks)
        const int c0 = split * a.split_keys, c1 = c0 + a.split_keys;
        const int j0 = max(jbeg, c0), j1 = min(jbeg + nblk * BN, c1);
        nblk = j1 > j0 ? (j1 - j0) / BN : 0;
        jbeg = j0;
        kend = min(Lk, c1);
    }
    // Key blocks run from the last to the first under ALiBi: scores fall with
    // the distance to the diagonal, so the first block holds the row maxima
    // and later blocks rarely move them (no O rescales).  Block it of the
    // walk, it = 0 .. nblk-1; it = nblk, nblk+1 (the pipelined prefetch past
    // the walk) fall outside [jbeg, jbeg + nblk*BN) and load nothing.
    const bool rev = BIAS && DP > 64 && MFA_ALIBI_REVERSE && a.alibi != nullptr;
    const int jfirst = rev ? jbeg + (nblk - 1) * BN : jbeg, jstep = rev ? -BN : BN;
    auto blk = [&](int it) { return jfirst + it * jstep; };
    const int wlast = min(wq0 + QB * 32, Lq) - 1;  // < wq0 when the wave has no rows
    const bool wave_live = wlast >= wq0;
    const int w_lo_first = key_lo(a, wq0 + dq), w_lo_last = key_lo(a, wlast + dq);
    const int w_hi_first = key_hi(a, wq0 + dq, Lk), w_hi_last = key_hi(a, wlast + dq, Lk);

    // ---- K/V streaming: global -> registers (block j+1) -> LDS buffer.
    // Buffer loads through a per-block resource whose size ends at the last
    // valid key row: rows past the sequence read as zero in hardware, and a
    // chunk past the head dim gets an offset beyond the resource (zero too),
    // so the loads carry no per-chunk conditions and no 64-bit address math.
    // At head dims 32 and 64 the threads cover whole rows: a lane's chunks
    // i = 0..KCH-1 share one column and sit RSTEP rows apart, so only chunk
    // 0's offsets are kept and the others are formed in the loop from
    // uniform row steps (the registers of KCH-1 offsets per operand are free
    // for the rest of the kernel: without them the D = 64 two-block tile
    // spilled 16-20 bytes, with a reload inside the loop).  A lane past the
    // head dim keeps an offset >= 2^31 for every chunk (the row steps stay
    // below 2^31: the planner bounds 63 rows of a stride to 2 GiB), so it
    // still reads zeros.  Not at head dim 128, which does not spill and whose
    // VALU-bound biased tiles measured 1 % slower with the in-loop adds.
    constexpr bool kRowStep = DP <= 64 && (kThreads % CPR == 0) && (KCH * kThreads == BN * CPR);
    constexpr int RSTEP = kThreads / CPR;
    u32x4_t kreg[KCH], vreg[KCH];
    uint32_t koff[KCH], voff[KCH];
    int lds_off[KCH], vlds_off[KCH];
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
        const int cc = tid + kThreads * i;
        const int row = cc / CPR, col = (cc % CPR) * 8;
        const bool in = (cc < BN * CPR) && (col < D);
        koff[i] = in ? (uint32_t)(((int64_t)row * a.ks + col) * 2) : 0x80000000u;
        voff[i] = in ? (uint32_t)(((int64_t)row * a.vs + col) * 2) : 0x80000000u;
        lds_off[i] = (cc < BN * CPR) ? row * KST + col : -1;
        vlds_off[i] = (cc < BN * CPR) ? row * VST + col : -1;
    }
    const uint32_t kstep = (uint32_t)(RSTEP * a.ks * 2), vstep = (uint32_t)(RSTEP * a.vs * 2);
    auto gload = [&](int j0) {
        // rows <= 0 (a block past the sequence, loaded branch-free by the
        // pipelined path) or a block before jbeg (past a reversed walk) gives
        // an empty resource: every lane reads zero (computed without
        // branches, so the pipelined block stays one basic block; the
        // address is formed from a block inside the range)
        const int j = max(j0, jbeg);
        const int rows = kend - j;
        const int rm1 = min(max(rows, 1), BN) - 1;
        bool kok, vok;
        const int64_t kbo = kv_block_off<PAGED>(a, sv, j, kend, a.kb, a.ks, kok);
        const int64_t vbo = kv_block_off<PAGED>(a, sv, j, kend, a.vb, a.vs, vok);
        const int live = -(int)(rows > 0 && j0 >= jbeg && kok && vok);
        // (readfirstlane: the sizes are uniform, but the clamp above selects
        // a vector med3, and a resource the backend sees in vector registers
        // gets a waterfall loop around every load)
        const int kbytes = __builtin_amdgcn_readfirstlane((int)(((int64_t)rm1 * a.ks + D) * 2) & live);
        const int vbytes = __builtin_amdgcn_readfirstlane((int)(((int64_t)rm1 * a.vs + D) * 2) & live);
        const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(sv.k + kbo * 2), (short)0, kbytes, kBufferDword3);
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(sv.v + vbo * 2), (short)0, vbytes, kBufferDword3);
        if constexpr (kRowStep && KCH > 1) {
            // (pinned copies: the per-chunk offsets are formed here, in the
            // loop, not hoisted out of it as KCH live registers)
            uint32_t k0 = koff[0], v0 = voff[0];
            pin(k0);
            pin(v0);
#pragma unroll
            for (int i = 0; i < KCH; ++i) {
                kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, k0 + i * kstep, 0, 0);
                vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, v0 + i * vstep, 0, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < KCH; ++i) {
                kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, koff[i], 0, 0);
                vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, voff[i], 0, 0);
            }
        }
    };
    auto swrite = [&](int buf) {
        uint16_t* kbuf = smem + buf * K_ELEMS;
        uint16_t* vbuf = smem + 2 * K_ELEMS + buf * V_ELEMS;
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            // (whole rows: chunk i is RSTEP rows below chunk 0, a constant
            // LDS offset)
            const int ko = kRowStep ? lds_off[0] + i * RSTEP * KST : lds_off[i];
            const int vo = kRowStep ? vlds_off[0] + i * RSTEP * VST : vlds_off[i];
            if (KCH * kThreads == BN * CPR || lds_off[i] >= 0) {
                *reinterpret_cast<u32x4_t*>(kbuf + ko) = kreg[i];
                *reinterpret_cast<u32x4_t*>(vbuf + vo) = vreg[i];
            }
        }
    };
    // PV A operand (V^T rows d = 32*db + lane%32, the 8 keys this half-wave's
    // accumulator registers 8*st..8*st+7 hold) from row-major V with two
    // ds_read_b64_tr_b16: in each 16-lane group, lane i addresses 4 elements
    // of key row (i/4) and lane j receives element j of rows 0..3.
    typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
    typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4_t;
    const int tr_row = 4 * half + ((lane & 15) >> 2);
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    auto load_vf = [&](const uint16_t* vbuf, int db, int kb, int st) -> op_t {
        const uint16_t* p0 = vbuf + (32 * kb + 16 * st + tr_row) * VST + 32 * db + tr_col;
        const uint16_t* p1 = p0 + 8 * VST;
        if constexpr (IS_BF16) {
            typedef __attribute__((address_space(3))) bf16x4_t* lp;
            const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lp)(p0));
            const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lp)(p1));
            return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        } else {
            typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 fp16x4_t;
            typedef __attribute__((address_space(3))) fp16x4_t* lp;
            const f16x4_t lo = __builtin_bit_cast(f16x4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lp)(p0)));
            const f16x4_t hi = __builtin_bit_cast(f16x4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lp)(p1)));
            return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    };
    auto mfma16 = [](const op_t& x, const op_t& y, const f32x16_t& acc) {
        if constexpr (IS_BF16)
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, acc, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(x, y, acc, 0, 0, 0);
    };

    // Sequential block: all QK^T, then per query block transform/max/update
    // (rescale only when some row's max moved) and probs, then all PV.
    auto block_simple = [&](auto masked_tag, const uint16_t* kbuf, const uint16_t* vtb, int j) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        f32x16_t sacc[QB][NKB];
        if constexpr (MFA_SIMPLE_PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                for (int r = 0; r < 16; ++r) sacc[qb][kb][r] = 0.f;
#pragma unroll
            for (int s = 0; s < DS; ++s) {
                const op_t kf = *reinterpret_cast<const op_t*>(kbuf + (32 * kb + l32) * KST + 16 * s + 8 * half);
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = mfma16(kf, qf[qb][s], sacc[qb][kb]);
            }
        }
        if constexpr (MFA_SIMPLE_PRIO) __builtin_amdgcn_s_setprio(0);
        u32x4_t pw[QB][NKB][2];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            qb_transform<NKB, BIAS, MASKED>(a, sacc[qb], rs[qb], j, half);
            float alpha;
            if (qb_update(rs[qb], qb_max<NKB>(sacc[qb]), c, tau_c, alpha)) scale_rows<DB>(o[qb], alpha);
            qb_probs16<NKB, IS_BF16>(sacc[qb], pw[qb], rs[qb].l, rs[qb].mu, c);
        }
        if constexpr (MFA_SIMPLE_PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const op_t vf = load_vf(vtb, db, kb, st);
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb)
                        o[qb][db] = mfma16(vf, __builtin_bit_cast(op_t, pw[qb][kb][st]), o[qb][db]);
                }
        if constexpr (MFA_SIMPLE_PRIO) __builtin_amdgcn_s_setprio(0);
    };

    // Block of the exact-row instantiation: query blocks one at a time, each
    // skipped when it holds no row of the sequence (a single query row leaves
    // every block but the wave's first empty), with two-term probabilities
    // and two PV MFMAs per V fragment (probs16x2_group).
    auto block_exact = [&](auto masked_tag, const uint16_t* kbuf, const uint16_t* vtb, int j) {
        constexpr bool MASKED = decltype(masked_tag)::value;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            if (wq0 + 32 * qb >= Lq) break;  // (wave-uniform)
            f32x16_t sacc[NKB];
            if constexpr (MFA_SIMPLE_PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
#pragma unroll
                for (int s = 0; s < DS; ++s) {
                    const op_t kf = *reinterpret_cast<const op_t*>(kbuf + (32 * kb + l32) * KST + 16 * s + 8 * half);
                    sacc[kb] = mfma16(kf, qf[qb][s], sacc[kb]);
                }
            }
            if constexpr (MFA_SIMPLE_PRIO) __builtin_amdgcn_s_setprio(0);
            qb_transform<NKB, BIAS, MASKED>(a, sacc, rs[qb], j, half);
            float alpha;
            if (qb_update(rs[qb], qb_max<NKB>(sacc), c, tau_c, alpha)) scale_rows<DB>(o[qb], alpha);
            // each group of 8 weights goes to the PV MFMAs right after it is
            // formed, so the scores free their registers group by group (the
            // lo terms would not fit beside all of them at head dim 128);
            // every O row block still sees the k-steps in the order
            // (kb, st), hi before lo
            float acc[2] = {0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    // (fenced, so the scheduler does not hoist every group's V
                    // fragment reads to the top, which would hold them all in
                    // registers at once)
                    __builtin_amdgcn_sched_barrier(0);
                    u32x4_t ph, pl;
                    probs16x2_group<IS_BF16>(sacc[kb], st, ph, pl, acc, rs[qb].mu, c);
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        const op_t vf = load_vf(vtb, db, kb, st);
                        o[qb][db] = mfma16(vf, __builtin_bit_cast(op_t, ph), o[qb][db]);
                        o[qb][db] = mfma16(vf, __builtin_bit_cast(op_t, pl), o[qb][db]);
                    }
                }
            __builtin_amdgcn_sched_barrier(0);
            rs[qb].l += acc[0] + acc[1];
        }
    };

    // Software-pipelined unmasked block (QB >= 2).  Program order:
    //   QK(0) | QK(1) + softmax(0) | PV(0) + softmax(1) | ... | PV(QB-1)
    // where "+" means the MFMAs are issued one or two at a time between the
    // chunks of the softmax (partial row max, running-max update, O rescale,
    // 8-probability groups), each chunk fenced by sched_barrier so the
    // compiler keeps the interleave: every MFMA then runs on the matrix core
    // while the following softmax chunk runs on the vector ALU.
    auto block_pipelined = [&](const uint16_t* kbuf, const uint16_t* vtb, int j, auto&& tail) {
        constexpr int kQK = NKB * DS;      // MFMAs of one QK^T
        constexpr int kPV = DB * NKB * 2;  // MFMAs of one PV
        constexpr int NCH = NKB + 1 + DB + 2 * NKB;  // softmax chunks
        op_t kf[NKB][DS];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int s = 0; s < DS; ++s)
                kf[kb][s] = *reinterpret_cast<const op_t*>(kbuf + (32 * kb + l32) * KST + 16 * s + 8 * half);
        f32x16_t sacc[QB][NKB];
        u32x4_t pw[QB][NKB][2];
        op_t vf[DB][NKB][2];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) sacc[qb][kb][r] = 0.f;
        // MFMA number mi of the group issued beside softmax(qb):
        // first the QK^T of query block qb+1, then the PV of query block qb-1
        auto issue = [&](int qb, int mi) {
            if (qb + 1 < QB) {
                if (mi < kQK) {
                    const int kb = mi / DS, s = mi % DS;
                    sacc[qb + 1][kb] = mfma16(kf[kb][s], qf[qb + 1][s], sacc[qb + 1][kb]);
                    return;
                }
                mi -= kQK;
            }
            if (qb > 0) {
                const int db = mi / (2 * NKB), kb = (mi / 2) % NKB, st = mi % 2;
                o[qb - 1][db] = mfma16(vf[db][kb][st], __builtin_bit_cast(op_t, pw[qb - 1][kb][st]), o[qb - 1][db]);
            }
        };
        if constexpr (MFA_SETPRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int s = 0; s < DS; ++s) sacc[0][kb] = mfma16(kf[kb][s], qf[0][s], sacc[0][kb]);
        if constexpr (MFA_SETPRIO) __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int st = 0; st < 2; ++st) vf[db][kb][st] = load_vf(vtb, db, kb, st);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const int nm = (qb + 1 < QB ? kQK : 0) + (qb > 0 ? kPV : 0);
            qb_transform<NKB, BIAS, false>(a, sacc[qb], rs[qb], j, half);
            float mpart[2] = {-INFINITY, -INFINITY}, alpha = 1.f;
            float lacc[2] = {0.f, 0.f};
            bool moved = false;
#pragma unroll
            for (int ci = 0; ci < NCH; ++ci) {
#pragma unroll
                for (int mi = ci * nm / NCH; mi < (ci + 1) * nm / NCH; ++mi) issue(qb, mi);
                if (ci < NKB) {  // partial row max over key block ci
#pragma unroll
                    for (int r = 0; r < 16; r += 2) {
                        mpart[0] = fmax_nn(mpart[0], sacc[qb][ci][r]);
                        mpart[1] = fmax_nn(mpart[1], sacc[qb][ci][r + 1]);
                    }
                } else if (ci == NKB) {  // merge halves, new running max
                    moved = qb_update(rs[qb], max_halves(fmax_nn(mpart[0], mpart[1])), c, tau_c, alpha);
                } else if (ci < NKB + 1 + DB) {  // rescale O rows (only if some row's max moved)
                    const int db = ci - NKB - 1;
                    if (moved) {
#pragma unroll
                        for (int r = 0; r < 16; ++r) o[qb][db][r] *= alpha;
                    }
                } else {  // 8 probabilities of (kb, st)
                    const int g = ci - NKB - 1 - DB, kb = g / 2, st = g % 2;
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        const float p0 = fast_exp2(fmaf(sacc[qb][kb][8 * st + 2 * w], c, -rs[qb].mu));
                        const float p1 = fast_exp2(fmaf(sacc[qb][kb][8 * st + 2 * w + 1], c, -rs[qb].mu));
                        pw[qb][kb][st][w] = pack_and_sum<IS_BF16>(p0, p1, lacc[w & 1]);
                    }
                    // (the block's sum joins l at the end, as in qb_probs16)
                    if (ci == NCH - 1) rs[qb].l += lacc[0] + lacc[1];
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // last PV: the K/V staging of the next blocks (LDS stores, global
        // loads) is issued between its MFMAs, which then run underneath it
        if constexpr (MFA_SETPRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int mi = 0; mi < kPV; ++mi) {
            issue(QB, mi);
            if (mi == 0) tail();
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (MFA_SETPRIO) __builtin_amdgcn_s_setprio(0);
    };

    // the first K/V block's global loads run while Q is staged
    if (nblk > 0) gload(blk(0));

    // ---- Q tile -> LDS (coalesced) -> registers as MFMA B operands (every
    // chunk of this thread loaded before any is stored: one memory round
    // trip, not one per chunk)
    {
        constexpr int QCH = (BM * CPR + kThreads - 1) / kThreads;  // chunks per thread
        u32x4_t val[QCH];
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
            const int c = tid + kThreads * i;
            const int row = c / CPR, col = (c % CPR) * 8;
            const int h = row / PM, pos = q0 + row - h * PM;
            val[i] = u32x4_t{0, 0, 0, 0};
            if (c < BM * CPR && pos < Lq && col < D)
                val[i] = *reinterpret_cast<const u32x4_t*>(sv.q + ((int64_t)h * a.qh1 + (int64_t)pos * a.qs + col) * 2);
        }
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
            const int c = tid + kThreads * i;
            if (QCH * kThreads == BM * CPR || c < BM * CPR)
                *reinterpret_cast<u32x4_t*>(smem + (c / CPR) * KST + (c % CPR) * 8) = val[i];
        }
    }
    __syncthreads();
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int s = 0; s < DS; ++s)
            qf[qb][s] = *reinterpret_cast<const op_t*>(smem + (wave * QB * 32 + qb * 32 + l32) * KST + 16 * s + 8 * half);
    __syncthreads();

    // Block it is computed from LDS buffer it%2 while the registers hold
    // block it+1 (loaded during block it-1): its LDS stores and the global
    // loads of block it+2 are issued during block it, one barrier per block.
    // (block 0's loads were issued before the Q tile was staged)
    if (nblk > 0) {
        swrite(0);
        if (nblk > 1) gload(blk(1));
        __syncthreads();
    }
    for (int it = 0; it < nblk; ++it) {
        const int j = blk(it);
        const int buf = it & 1;
        auto stage_next = [&]() {
            if (it + 1 < nblk) swrite(buf ^ 1);
            if (it + 2 < nblk) gload(blk(it + 2));
        };
        const bool skip = !wave_live || (j + BN - 1 < w_lo_first) || (j > w_hi_last);
        const bool masked = !((j >= w_lo_last) && (j + BN - 1 <= w_hi_first));
        const uint16_t* kbuf = smem + buf * K_ELEMS;
        const uint16_t* vtb = smem + 2 * K_ELEMS + buf * V_ELEMS;  // row-major V
        if constexpr (EXACT) {
            if (!skip) {
                if (masked)
                    block_exact(std::true_type{}, kbuf, vtb, j);
                else
                    block_exact(std::false_type{}, kbuf, vtb, j);
            }
            stage_next();
        } else if (QB >= 2 && MFA_PIPELINE && !skip && !masked) {
            if constexpr (QB >= 2 && MFA_PIPELINE) {
                if constexpr (MFA_STAGE_IN_PV && MFA_BRANCHFREE_STAGE) {
                    // unconditional staging: no branch splits the pipelined
                    // block, so no softmax work is sunk below the staging.
                    // Past the last block it writes the idle buffer and loads
                    // through an empty resource (no memory access).
                    block_pipelined(kbuf, vtb, j, [&]() {
                        swrite(buf ^ 1);
                        gload(blk(it + 2));
                    });
                } else if constexpr (MFA_STAGE_IN_PV) {
                    block_pipelined(kbuf, vtb, j, stage_next);
                } else {
                    block_pipelined(kbuf, vtb, j, [] {});
                    stage_next();
                }
            }
        } else {
            if (!skip) {
                if (masked)
                    block_simple(std::true_type{}, kbuf, vtb, j);
                else
                    block_simple(std::false_type{}, kbuf, vtb, j);
            }
            stage_next();
        }
        __syncthreads();
    }

    if (a.nsplit > 1) {
        store_partial<QB, DB>(a, Lq, b * a.Hq + hq, split, o, rs, c, wq0, lane);
    } else {  // (the loop's last barrier released the LDS)
        SeqView svh = sv;  // this wave's head: its O and lse rows
        if (!EXACT && hl != 0) {
            svh.o += (int64_t)hl * a.oh1 * (a.out_f32 ? 4 : 2);
            if (svh.lse) svh.lse += (int64_t)hl * a.lse_h1;
        }
        store_out_rows<QB, DB, IS_BF16, KST>(a, svh, o, rs, wq0, lane, c,
                                             smem + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * QB * 32 * KST);
    }
}

// ----------------------------------------------------------------------------
// 16-bit ping-pong kernel.
//
// Eight wavefronts in two groups of four, one wavefront of each group per
// SIMD (grouped at start-up by the SIMD each one landed on).  Each wavefront
// owns QB 32-query blocks (two for head dims up to 64, one above) and
// alternates two phases:
//   A(t): PV(t-1) then QK(t)        -- MFMAs only (32 for d64 x2, d128 x1)
//   B(t): softmax of S(t)           -- VALU only
// The groups run a phase apart, one workgroup barrier between phases, so on
// every SIMD one wavefront keeps the matrix core busy while the other keeps the
// vector ALU busy, and every operand a phase needs was produced by the phase
// before it.  K/V tiles arrive by direct-to-LDS loads (one instruction
// writes 64 x 16 bytes contiguously, lane i at 16*i, from a per-lane source
// offset; no staging registers or LDS store instructions) into three stages
// per operand: K(t) is read in both groups' A(t), V(t) in both groups'
// A(t+1); each even phase 2u issues the loads of K(u+2) and V(u+1) into
// stages the previous barrier released.  Tiles are unpadded with the 16-byte
// chunks of each row XOR-swizzled, so the K operand reads (one row per lane)
// and the transposed V reads (four rows per 16 lanes) are free of bank
// conflicts.
// steps of one MFMA phase of the ping-pong kernel
constexpr int kBothHalves = 0, kQkOnly = 1, kPvOnly = 2;

template <int DP, int QB, int NKB, bool IS_BF16, bool BIAS, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW / 4)))
mfa_fwd16_pp_kernel(KArgs a) {
    static_assert(NW == 8 || NW == 16, "two or four wavefronts per SIMD");
    constexpr bool SUM_IN_A = MFA_PP_SUM_IN_A;
    // the first and last MFMA phases run their real half only (head dim 128:
    // config 4 -1.5 %, config 3 -0.7 %; at 64 the code grew slower by 0.4 %)
    constexpr bool TRIM = DP > 64;
    constexpr int NT = NW * 64;        // threads
    constexpr int BM = NW * QB * 32;   // query rows per workgroup
    constexpr int BN = NKB * 32;       // keys per K/V block
    constexpr int DS = DP / 16;
    constexpr int DB = DP / 32;
    constexpr int NST = 3;             // LDS stages per operand
    constexpr int CPR = DP / 8;        // 16-byte chunks per row
    constexpr int TILE = BN * DP;      // elements of one K or V tile
    constexpr int KV_ELEMS = 2 * NST * TILE;
    constexpr int KST = DP + 8;        // Q staging row stride
    constexpr int Q_ELEMS = BM * KST;
    constexpr int SMEM = KV_ELEMS > Q_ELEMS ? KV_ELEMS : Q_ELEMS;
    constexpr int TI = BN * CPR / 64;  // 1 KiB wave loads per tile
    // every loading wavefront issues NL loads per tile (waves >= TI none)
    constexpr int NL = TI >= NW ? TI / NW : 1;
    static_assert(BN * CPR % 64 == 0 && (TI < NW || TI % NW == 0), "equal load counts per wavefront");
    typedef typename std::conditional<IS_BF16, bf16x8_t, f16x8_t>::type op_t;

    __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM];
    __shared__ int simd_count[4];

    int b, hq, tile;
    if (!decode_tile(a, blockIdx.x, b, hq, tile)) return;
    const SeqView sv = seq_view<2>(a, b, hq);
    // Head-packed tiles (a.hpack > 1): the tile holds PM positions of each of
    // hpack query heads of one K/V head, head-major (tile row = head * PM +
    // position), so wave w takes head w / (NW / hpack) at position block
    // w % (NW / hpack) and every wave reads its rows at LDS row w * QB * 32.
    const int hpk = a.hpack;
    const int PM = BM / hpk;  // positions per tile
    const int q0 = tile * PM;
    if (q0 >= sv.Lq) return;
    if (a.single_rows != 0 && sv.Lq == 1) return;  // (the exact-row kernel's launch computes it)

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, half = lane >> 5;
    const int Lq = sv.Lq, Lk = sv.Lk, D = a.D;
    const int dq = Lk - Lq;
    const int wph = NW / hpk;                  // waves per head
    const int hl = wave / wph;                 // this wave's head inside the tile
    const int wq0 = q0 + (wave - hl * wph) * QB * 32;  // first position of this wavefront

    // ---- Q tile -> LDS (coalesced) -> registers as MFMA B operands.  Every
    // chunk of this thread is loaded before any is stored: as one loop the
    // compiler waited for each load before its LDS store, one memory round
    // trip per chunk (measured ~15,000 cycles per tile for 8 chunks).
    if (tid < 4) simd_count[tid] = 0;
    {
        constexpr int QCH = (BM * CPR + NT - 1) / NT;  // chunks per thread
        u32x4_t val[QCH];
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
            const int c = tid + NT * i;
            const int row = c / CPR, col = (c % CPR) * 8;
            const int h = row / PM, pos = q0 + row - h * PM;
            val[i] = u32x4_t{0, 0, 0, 0};
            if (c < BM * CPR && pos < Lq && col < D)
                val[i] = *reinterpret_cast<const u32x4_t*>(sv.q + ((int64_t)h * a.qh1 + (int64_t)pos * a.qs + col) * 2);
        }
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
            const int c = tid + NT * i;
            if (QCH * NT == BM * CPR || c < BM * CPR)
                *reinterpret_cast<u32x4_t*>(smem + (c / CPR) * KST + (c % CPR) * 8) = val[i];
        }
    }
    __syncthreads();
    op_t qf[QB][DS];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int s = 0; s < DS; ++s)
            qf[qb][s] = *reinterpret_cast<const op_t*>(smem + (wave * QB * 32 + qb * 32 + l32) * KST + 16 * s + 8 * half);
    // group: the order in which the wavefronts of one SIMD arrive (SIMD_ID =
    // HW_ID[5:4]); the grouping only affects speed, never results
    int arrival = 0;
    if (lane == 0) arrival = atomicAdd(&simd_count[__builtin_amdgcn_s_getreg((1 << 11) | (4 << 6) | 4)], 1);
    const int grp = __builtin_amdgcn_readfirstlane(arrival) & 1;
    __syncthreads();

    RowState rs[QB];
    int lo_max[QB], hi_min[QB];  // per query block: largest lower / smallest upper key bound
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        rs[qb].center = wq0 + 32 * qb + l32 + dq;
        rs[qb].lo = key_lo(a, rs[qb].center);
        rs[qb].hi = key_hi(a, rs[qb].center, Lk);
        rs[qb].slope = a.alibi ? a.alibi[b * a.alibi_bstride + hq * hpk + hl] : 0.f;
        row_reset(rs[qb]);
        const int r0 = wq0 + 32 * qb;
        const int r1 = max(min(r0 + 31, Lq - 1), r0);
        lo_max[qb] = key_lo(a, r1 + dq);
        hi_min[qb] = key_hi(a, r0 + dq, Lk);
    }
    f32x16_t o[QB][DB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[qb][db][r] = 0.f;
    const float c = BIAS ? kLog2e : a.scale_log2;
    // per-row rescales for single-row sequences, as in the 4-wavefront kernel
    // (the two kernels then agree bit for bit on every shape)
    const float tau = Lq == 1 ? 0.f : (float)MFA_RESCALE_TAU;
    const float tau_c = tau / c;

    // this wave's head: its O and lse rows
    SeqView svh = sv;
    svh.o += (int64_t)hl * a.oh1 * (a.out_f32 ? 4 : 2);
    if (svh.lse) svh.lse += (int64_t)hl * a.lse_h1;

    // ---- key range of the workgroup
    const int qlast = min(q0 + PM, Lq) - 1;
    const int klo = key_lo(a, q0 + dq);
    const int khi = key_hi(a, qlast + dq, Lk);
    const int jbeg = (klo / BN) * BN;
    const int nblk = khi >= klo ? (khi - jbeg) / BN + 1 : 0;
    if (nblk == 0) {  // no valid key for any row of the tile: zeros
        store_out<QB, DB, IS_BF16>(a, svh, o, rs, wq0, lane, c);
        return;
    }
    // key block of step u, last block first under ALiBi (as in the
    // 4-wavefront kernel); steps past the walk load nothing
    const bool rev = BIAS && DP > 64 && MFA_ALIBI_REVERSE && a.alibi != nullptr;
    const int jfirst = rev ? jbeg + (nblk - 1) * BN : jbeg, jstep = rev ? -BN : BN;
    auto blk = [&](int u) { return jfirst + u * jstep; };

    // ---- LDS tiles: chunk c of row r is stored in chunk slot c ^ swz(r).
    // The LDS serves 256 bytes per cycle: the 16 lanes of one ds_read_b128
    // cycle (one K row each, the same chunk index) and the 32 lanes of one
    // ds_read_b64_tr_b16 cycle (4 V rows x 64 bytes) must fall in distinct
    // 16-byte bank groups of a 256-byte line (SQ_LDS_BANK_CONFLICT = 0
    // measured at head dims 64 and 128).  Rows are 256, 128 or 64 bytes:
    // 1, 2 or 4 rows share a line, so the swizzle spreads rows that share
    // a line position.
    auto kswz = [](int r) {
        if constexpr (CPR == 16) return r & 15;
        else if constexpr (CPR == 8) return (r >> 1) & 7;
        else return (r >> 2) & 3;
    };
    auto vswz = [](int r) {  // 4-chunk groups stay contiguous (multiples of 4)
        if constexpr (CPR == 16) return 4 * (r & 3);
        else if constexpr (CPR == 8) return 4 * ((r >> 1) & 1);
        else return 0;
    };
    uint16_t* const kst0 = smem;
    uint16_t* const vst0 = smem + NST * TILE;
    // direct-to-LDS loads: load i of wave w fills tile slots
    // 64*(w + NW*i) .. +63 (w < TI when a tile is smaller than NW loads)
    const bool loader = TI >= NW || wave < TI;
    uint32_t kdoff[NL], vdoff[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int s = 64 * (wave + NW * i) + lane;
        const int r = s / CPR, p = s % CPR;
        const int ck = p ^ kswz(r), cv = p ^ vswz(r);
        kdoff[i] = loader && ck * 8 < D ? (uint32_t)(((int64_t)r * a.ks + ck * 8) * 2) : 0x80000000u;
        vdoff[i] = loader && cv * 8 < D ? (uint32_t)(((int64_t)r * a.vs + cv * 8) * 2) : 0x80000000u;
    }
    // Buffer resource of K/V block u: base + j*stride bytes, sized to the
    // block's valid rows (min(BN, Lk - j); none past the sequence).  All
    // fields are wave-uniform and computed with scalar arithmetic (the
    // host bounds the block span to 31 bits).
    const int kfull = ((BN - 1) * (int)a.ks + D) * 2;
    const int vfull = ((BN - 1) * (int)a.vs + D) * 2;
    auto load_block = [&](const char* base, int64_t bstride, int64_t stride, int full, uint16_t* dst, uint32_t off,
                          int u) __attribute__((always_inline)) {
        const int j0 = blk(u), j = max(j0, jbeg);
        const int rows = Lk - j;
        bool ok;
        const int64_t bo = kv_block_off<false>(a, sv, j, Lk, bstride, stride, ok);
        int bytes = full;
        if (rows < BN) bytes = rows > 0 ? ((rows - 1) * (int)stride + D) * 2 : 0;
        // steps past the walk load nothing (under causal masks their blocks
        // can lie inside the sequence, and their reads would be wasted)
        if (!ok || j0 < jbeg || u >= nblk) bytes = 0;
        lds_load16(reinterpret_cast<uint64_t>(base + bo * 2), (uint32_t)bytes, dst, off);
    };
    // loads of K block u into its stage u % NST (and likewise V); wave-uniform
    auto load_k = [&](int u) __attribute__((always_inline)) {
        if (loader) {
#pragma unroll
            for (int i = 0; i < NL; ++i)
                load_block(sv.k, a.kb, a.ks, kfull, kst0 + (u % NST) * TILE + 512 * (wave + NW * i), kdoff[i], u);
        }
    };
    auto load_v = [&](int u) __attribute__((always_inline)) {
        if (loader) {
#pragma unroll
            for (int i = 0; i < NL; ++i)
                load_block(sv.v, a.vb, a.vs, vfull, vst0 + (u % NST) * TILE + 512 * (wave + NW * i), vdoff[i], u);
        }
    };
    // Barrier at the end of phase p, once this wave's LDS reads have returned
    // and the loads the next phase reads have landed.  Phase p+1 reads the
    // batch issued at phase p-3 (p odd) or p-4 (p even), so the newest one
    // (p odd) or two (p even) batches of 2*NL loads may still be in flight.
    auto phase_sync = [&](auto even_c) {
        if constexpr (decltype(even_c)::value)
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(4 * NL) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(2 * NL) : "memory");
    };

    // ---- MFMA operand reads.  K operand: row 32*kb + l32, chunk 2*s + half
    // (rows 32*kb + l32 share the swizzle bits of l32).  PV A operand (V^T
    // rows d = 32*db + lane%32, the 8 keys of accumulator registers
    // 8*st..8*st+7) with two ds_read_b64_tr_b16: in each 16-lane group, lane
    // i addresses 4 elements of key row (i/4) and lane j receives element j
    // of rows 0..3.
    // Per-lane element offsets, swizzle included, of the fragments that differ
    // only in their lane part: K step s, V head-dim block db.  The key-block
    // and row-group parts are compile-time constants (immediate offsets).
    const int kz = kswz(l32);
    int klane[DS];
#pragma unroll
    for (int s = 0; s < DS; ++s) klane[s] = l32 * DP + 8 * ((2 * s + half) ^ kz);
    auto load_kf = [&](const uint16_t* const (&kp)[DS], int kb, int s) -> op_t {
        return *reinterpret_cast<const op_t*>(kp[s] + 32 * kb * DP);
    };
    const int tr_row = 4 * half + ((lane & 15) >> 2);
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int vz = vswz(tr_row);
    int vlane[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) vlane[db] = tr_row * DP + 8 * ((4 * db + (tr_col >> 3)) ^ vz) + (tr_col & 7);
    auto mfma16 = [](const op_t& x, const op_t& y, const f32x16_t& acc) {
        if constexpr (IS_BF16)
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, acc, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(x, y, acc, 0, 0, 0);
    };

    f32x16_t sacc[QB][NKB];  // S^T(t) of query block qb
    u32x4_t pw[QB][NKB][2];  // 16-bit P^T(t), PV B operands

    // A(u): PV(u-1) then QK(u).  Step i reads one K or V
    // fragment, which feeds both query blocks; fragments are read
    // MFA_PP_AHEAD steps ahead of their MFMAs (sched_barrier keeps the
    // compiler from hoisting every read to the top).  PART selects the
    // steps: both halves, the QK half only (A(0): block -1 has no P) or the
    // PV half only (A(n): block n has no scores to compute).
    auto phase_a = [&](int u, auto part_c) __attribute__((always_inline)) {
        constexpr int PART = decltype(part_c)::value;
        constexpr int NPV = DB * NKB * 2;
        constexpr int NQK = NKB * DS;
        constexpr int I0 = PART == kQkOnly ? NPV : 0;         // first step
        constexpr int NS = PART == kPvOnly ? NPV : NPV + NQK;  // end of the steps
        constexpr int AH = NW == 16 ? MFA_PP_AHEAD16 : QB == 1 ? (DP > 64 ? MFA_PP_AHEAD1W : MFA_PP_AHEAD1) : MFA_PP_AHEAD;
        const uint16_t* vt = vst0 + ((u + NST - 1) % NST) * TILE;
        const uint16_t* kt = kst0 + (u % NST) * TILE;
        const uint16_t* kp[DS];
        uint32_t vp[DB];
#pragma unroll
        for (int s = 0; s < DS; ++s) kp[s] = kt + klane[s];
        const uint32_t vt_lds = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)vt;
#pragma unroll
        for (int db = 0; db < DB; ++db) vp[db] = vt_lds + 2 * vlane[db];
        // step i: one V fragment (two transposed reads, issued from asm with
        // the row-group offset as an immediate) or one K fragment (compiler
        // load); fragments are read AH steps ahead of their MFMAs
        u32x2_t vlo[AH + 1], vhi[AH + 1];
        op_t kfr[AH + 1];
        auto load_step = [&](auto ic) __attribute__((always_inline)) {
            constexpr int i = decltype(ic)::value;
            if constexpr (i < I0) {
            } else if constexpr (i < NPV) {
                constexpr int db = i % DB, ks = i / DB, kb = ks / 2, st = ks % 2;
                constexpr int off = (32 * kb + 16 * st) * DP * 2;
                vlo[i % (AH + 1)] = lds_read_tr16<off>(vp[db]);
                vhi[i % (AH + 1)] = lds_read_tr16<off + 8 * DP * 2>(vp[db]);
            } else if constexpr (i < NS) {
                constexpr int m = i - NPV, kb = m % NKB, s = m / NKB;
                kfr[i % (AH + 1)] = load_kf(kp, kb, s);
            }
        };
        auto mfma_step = [&](auto ic) __attribute__((always_inline)) {
            constexpr int i = decltype(ic)::value;
            if constexpr (i < NPV) {
                // LDS operations issued after this step's reads (steps i+1 .. i+AH)
                constexpr int after = [] {
                    int n = 0;
                    for (int k = i + 1; k <= i + AH && k < NS; ++k) n += k < NPV ? 2 : 1;
                    return n;
                }();
                u32x2_t lo = vlo[i % (AH + 1)], hi = vhi[i % (AH + 1)];
                lds_wait<after>(lo, hi);
                const op_t f = __builtin_bit_cast(op_t, u32x4_t{lo[0], lo[1], hi[0], hi[1]});
                constexpr int db = i % DB, ks = i / DB, kb = ks / 2, st = ks % 2;
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
                    o[qb][db] = mfma16(f, __builtin_bit_cast(op_t, pw[qb][kb][st]), o[qb][db]);

            } else {
                const op_t f = kfr[i % (AH + 1)];
                constexpr int m = i - NPV, kb = m % NKB, s = m / NKB;
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
                    sacc[qb][kb] = mfma16(f, qf[qb][s], s == 0 ? f32x16_t{} : sacc[qb][kb]);
            }
        };
        if constexpr (MFA_PP_PRIO) __builtin_amdgcn_s_setprio(MFA_PP_PRIO);
        static_for<AH>([&](auto ic) __attribute__((always_inline)) {
            load_step(std::integral_constant<int, I0 + decltype(ic)::value>{});
        });
        if constexpr (SUM_IN_A && PART != kQkOnly) {
            // row sums of P(u-1), whose rescale (if any) B(u-1) applied to l
            // (the pins keep the compiler from moving the sums into B)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int st = 0; st < 2; ++st) pin(pw[qb][kb][st]);
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) rs[qb].l += qb_sum16<NKB, IS_BF16>(pw[qb]);
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) pin(rs[qb].l);
        }
        __builtin_amdgcn_sched_barrier(0);
        static_for<NS - I0>([&](auto ic) __attribute__((always_inline)) {
            constexpr int i = I0 + decltype(ic)::value;
            load_step(std::integral_constant<int, i + AH>{});
            mfma_step(std::integral_constant<int, i>{});
            __builtin_amdgcn_sched_barrier(0);
        });
        if constexpr (MFA_PP_PRIO) __builtin_amdgcn_s_setprio(0);
    };
    // B(u): online softmax of S(u) for both query blocks
    auto phase_b = [&](int u) __attribute__((always_inline)) {
        const int j = blk(u);
        // the softmax stays between the barriers: it starts from S as the
        // phase begins and its P is complete before the phase ends
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) pin(sacc[qb][kb]);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            if ((j >= lo_max[qb]) && (j + BN - 1 <= hi_min[qb]))
                qb_transform<NKB, BIAS, false>(a, sacc[qb], rs[qb], j, half);
            else
                qb_transform<NKB, BIAS, true>(a, sacc[qb], rs[qb], j, half);
        }
        // both query blocks' max, update and probabilities in one branch-free
        // stretch (independent chains for the scheduler to interleave); the
        // rare rescale of O follows (O is next read by PV in the next phase)
        float mx[QB], m_old[QB], bsum[QB];
        bool moved[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) mx[qb] = qb_max<NKB>(sacc[qb]);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) moved[qb] = qb_move(rs[qb], mx[qb], c, tau_c, m_old[qb]);
        if constexpr (SUM_IN_A) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                qb_probs16_only<NKB, IS_BF16>(sacc[qb], pw[qb], rs[qb].mu, c);
                bsum[qb] = 0.f;  // (added in the next MFMA phase)
            }
        } else if constexpr (MFA_PP_LATE_SUM && DP <= 64) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) qb_probs16_only<NKB, IS_BF16>(sacc[qb], pw[qb], rs[qb].mu, c);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) bsum[qb] = qb_sum16<NKB, IS_BF16>(pw[qb]);
        } else {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                bsum[qb] = 0.f;
                qb_probs16<NKB, IS_BF16>(sacc[qb], pw[qb], bsum[qb], rs[qb].mu, c);
            }
        }
        // the rare rescale of O and l: alpha only when the reference moved
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
            if (moved[qb]) {
                const float alpha = move_alpha(m_old[qb], rs[qb].m, c);
                scale_rows<DB>(o[qb], alpha);
                rs[qb].l *= alpha;
            }
        if constexpr (!SUM_IN_A) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) rs[qb].l += bsum[qb];
        }
        // (the row sums stay in this phase too)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) pin(rs[qb].l);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int st = 0; st < 2; ++st) pin(pw[qb][kb][st]);
    };
    // ---- prologue: K(0), K(1), V(0) resident.  With TRIM, A(0) runs only
    // the QK of block 0 and A(n) only the PV of block n-1; without, A(0) runs
    // PV(-1) with P = 0 against the zeroed V stage of block -1 and A(n) a QK
    // of block n whose result is never used.
    if constexpr (!TRIM) {
        for (int c2 = tid; c2 < TILE / 8; c2 += NT)
            *reinterpret_cast<u32x4_t*>(vst0 + (NST - 1) * TILE + 8 * c2) = u32x4_t{0, 0, 0, 0};
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int st = 0; st < 2; ++st) pw[qb][kb][st] = u32x4_t{0, 0, 0, 0};
    }
    load_k(0);
    load_k(1);
    load_v(0);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- phases: group 0 runs A(0) B(0) A(1) ... B(n-1) A(n) at phases
    // 0..2n, group 1 the same at phases 1..2n+1; every wave issues the loads
    // of K(u+2), V(u+1) at phase 2u (blocks past the end read zero).
    auto dma = [&](int u) __attribute__((always_inline)) {
        load_k(u + 2);
        load_v(u + 1);
    };
    using EVEN = std::true_type;
    using ODD = std::false_type;
    // With MFA_PP_DMA_A, group 1 issues its share of batch u at the start of
    // its own A(u) (phase 2u+1) instead of in its softmax phase B(u-1), where
    // the load issue sat on the critical path (the phase pairs A of group 0
    // with B of group 1).  Batch u is first read at phase 2u+4 and overwrites
    // stages last read at phase 2u-1, so issuing it at 2u+1 is safe; group 1
    // then keeps at most its newest batch in flight at every barrier.
    auto run = [&](auto grp_c) __attribute__((always_inline)) {
        constexpr int G = decltype(grp_c)::value;
        // (head dims up to 64 only: at 128 a block's loads need the extra phase)
        constexpr bool LATE = MFA_PP_DMA_A && G == 1 && DP <= 64;
        if constexpr (G == 1) {
            if constexpr (!LATE) dma(0);
            phase_sync(std::integral_constant<bool, !LATE>{});  // phase 0 (idle)
        }
        auto step = [&](int u, auto part_c) __attribute__((always_inline)) {
            if constexpr (G == 0 || LATE) dma(u);
            phase_a(u, part_c);
            if constexpr (G == 0) phase_sync(EVEN{}); else phase_sync(ODD{});
            if constexpr (G == 1 && !LATE) dma(u + 1);
            phase_b(u);
            if constexpr (G == 0) phase_sync(ODD{});
            else phase_sync(std::integral_constant<bool, !LATE>{});
        };
        if constexpr (TRIM) {
            step(0, std::integral_constant<int, kQkOnly>{});  // (nblk >= 1 here)
            for (int u = 1; u < nblk; ++u) step(u, std::integral_constant<int, kBothHalves>{});
        } else {
            for (int u = 0; u < nblk; ++u) step(u, std::integral_constant<int, kBothHalves>{});
        }
        if constexpr (G == 0 || LATE) dma(nblk);
        phase_a(nblk, std::integral_constant<int, TRIM ? kPvOnly : kBothHalves>{});
        if constexpr (G == 0) {
            phase_sync(EVEN{});  // phase 2n
            phase_sync(ODD{});   // phase 2n+1 (idle)
        } else {
            phase_sync(ODD{});   // phase 2n+1
        }
    };
    if (grp == 0)
        run(std::integral_constant<int, 0>{});
    else
        run(std::integral_constant<int, 1>{});
    // no direct-to-LDS write may land after the workgroup's LDS is released,
    // nor in the O blocks below (every wavefront's loads done, then a barrier)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    store_out_rows<QB, DB, IS_BF16, KST>(a, svh, o, rs, wq0, lane, c, smem + wave * QB * 32 * KST);
}

// ----------------------------------------------------------------------------
// 16-bit kernel for at most 32 keys per sequence (cross-attention to a short
// conditioning sequence: many query rows, a handful of keys).  The keys fit
// one 32-key block, so each wavefront keeps K and V^T as MFMA operands in
// registers (staged once through LDS, in the 4-wavefront kernel's layout)
// and streams NQ 32-row query blocks through them: Q fragments straight from
// global memory, S^T = K Q^T, the online softmax of a single block, O^T = V^T
// P^T, O stored.  No barrier after the set-up: the kernel moves Q in and O out
// (HBM-bound).  Per row it performs the 4-wavefront kernel's operations in
// its order (its second 32-key block and its second PV step add only zeros
// there), so both give the same bits.
#ifndef MFA_TK_BLOCKS
#define MFA_TK_BLOCKS 1
#endif
#ifndef MFA_TK
#define MFA_TK 1
#endif
// wavefronts per SIMD the tiny-key kernel is register-budgeted for
#ifndef MFA_TK_WAVES
#define MFA_TK_WAVES 3
#endif
// query rows from which the tiny-key kernel is chosen
#ifndef MFA_TK_MIN_ROWS
#define MFA_TK_MIN_ROWS 128
#endif
template <int DP, bool IS_BF16, bool BIAS>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(MFA_TK_WAVES)))
mfa_fwd16_tk_kernel(KArgs a) {
    constexpr int DS = DP / 16, DB = DP / 32;
    constexpr int NQ = MFA_TK_BLOCKS;          // 32-row query blocks per wavefront
    constexpr int BM = kWaves * NQ * 32;       // query rows per workgroup
    // LDS row stride (elements) of K, V and the Q / O blocks: +16 bytes
    // against bank conflicts in the row-per-lane reads (V is read once per
    // workgroup, so its transposed reads need no wider padding)
    constexpr int KST = DP + 8;
    constexpr int VST = KST;
    constexpr int CPR = DP / 8;                // 16-byte chunks per row
    typedef typename std::conditional<IS_BF16, bf16x8_t, f16x8_t>::type op_t;
    // K, V (at most 32 rows each) and one 32-row Q / O block per wavefront
    __shared__ __attribute__((aligned(16))) uint16_t kv_s[32 * KST + 32 * VST + kWaves * 32 * KST];
    uint16_t* const tk_s = kv_s + 32 * KST + 32 * VST;

    int b, hq, tile;
    if (!decode_tile(a, blockIdx.x, b, hq, tile)) return;
    const SeqView sv = seq_view<2>(a, b, hq);
    const int q0 = tile * BM;
    if (q0 >= sv.Lq) return;
    if (a.single_rows != 0 && sv.Lq == 1) return;  // (the exact-row kernel's launch computes it)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, half = lane >> 5;
    const int Lq = sv.Lq, Lk = sv.Lk, D = a.D;
    const int dq = Lk - Lq;

    // Q in and O out go through this wavefront's LDS block (32 rows), so that
    // global reads and writes are row-contiguous: 16 lanes cover a 256-byte
    // row (MFMA operand order would touch 32 rows in 16-32 byte pieces).  The
    // next block's rows are loaded into registers before this block's MFMAs,
    // the first block's during the K/V set-up.
    constexpr int QCH = 32 * CPR / 64;  // 16-byte chunks per lane and block
    uint16_t* const qo = tk_s + wave * (32 * KST);
    u32x4_t qn[QCH];
    // (buffer loads through a resource sized to the block's valid rows:
    // rows past the sequence and chunks past the head dim read zero, with no
    // branches, so the waits on them are counted exactly)
    auto load_q = [&](int n) __attribute__((always_inline)) {
        const int r0 = q0 + (wave * NQ + n) * 32;
        const int rows = min(Lq - r0, 32);
        const int bytes = __builtin_amdgcn_readfirstlane(rows > 0 ? (int)(((int64_t)(rows - 1) * a.qs + D) * 2) : 0);
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(sv.q + (int64_t)max(r0, 0) * a.qs * 2), (short)0, bytes, kBufferDword3);
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
            const int ch = lane + 64 * i, col = (ch % CPR) * 8;
            const uint32_t off = col < D ? (uint32_t)(((int64_t)(ch / CPR) * a.qs + col) * 2) : 0x80000000u;
            qn[i] = __builtin_amdgcn_raw_buffer_load_b128(qr, off, 0, 0);
        }
    };

    // ---- K and V rows (zero past the sequence and the head dim) -> LDS
    uint16_t* const vs = kv_s + 32 * KST;
    constexpr int KVC = (32 * CPR + kThreads - 1) / kThreads;  // chunks per thread
    u32x4_t kk[KVC], vv[KVC];
    {
        const int kbytes = __builtin_amdgcn_readfirstlane(Lk > 0 ? (int)(((int64_t)(Lk - 1) * a.ks + D) * 2) : 0);
        const int vbytes = __builtin_amdgcn_readfirstlane(Lk > 0 ? (int)(((int64_t)(Lk - 1) * a.vs + D) * 2) : 0);
        const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc((void*)sv.k, (short)0, kbytes, kBufferDword3);
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc((void*)sv.v, (short)0, vbytes, kBufferDword3);
#pragma unroll
        for (int i = 0; i < KVC; ++i) {
            const int ch = tid + kThreads * i, row = ch / CPR, col = (ch % CPR) * 8;
            const bool in = ch < 32 * CPR && col < D;
            kk[i] = __builtin_amdgcn_raw_buffer_load_b128(
                kr, in ? (uint32_t)(((int64_t)row * a.ks + col) * 2) : 0x80000000u, 0, 0);
            vv[i] = __builtin_amdgcn_raw_buffer_load_b128(
                vr, in ? (uint32_t)(((int64_t)row * a.vs + col) * 2) : 0x80000000u, 0, 0);
        }
    }
    load_q(0);  // (after the K/V loads: their results are waited for first)
#pragma unroll
    for (int i = 0; i < KVC; ++i) {
        const int ch = tid + kThreads * i, row = ch / CPR, col = (ch % CPR) * 8;
        if (KVC * kThreads == 32 * CPR || ch < 32 * CPR) {
            *reinterpret_cast<u32x4_t*>(kv_s + row * KST + col) = kk[i];
            *reinterpret_cast<u32x4_t*>(vs + row * VST + col) = vv[i];
        }
    }
    __syncthreads();
    // K operand: row l32, k-slots 16*s + 8*half.. ; V^T operand of PV step
    // st: the 4-wavefront kernel's transposed reads (lane i of a 16-lane group
    // addresses 4 elements of key row i/4, lane j receives element j of rows 0..3)
    op_t kf[DS], vf[DB][2];
#pragma unroll
    for (int s = 0; s < DS; ++s) kf[s] = *reinterpret_cast<const op_t*>(kv_s + l32 * KST + 16 * s + 8 * half);
    const int tr_row = 4 * half + ((lane & 15) >> 2);
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const uint16_t* p0 = vs + (16 * st + tr_row) * VST + 32 * db + tr_col;
            const uint16_t* p1 = p0 + 8 * VST;
            typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 fp16x4_t;
            typedef __attribute__((address_space(3))) fp16x4_t* lp;
            const u32x2_t lo = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lp)(p0)));
            const u32x2_t hi = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lp)(p1)));
            vf[db][st] = __builtin_bit_cast(op_t, u32x4_t{lo[0], lo[1], hi[0], hi[1]});
        }
    auto mfma16 = [](const op_t& x, const op_t& y, const f32x16_t& acc) {
        if constexpr (IS_BF16)
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, acc, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(x, y, acc, 0, 0, 0);
    };
    const float c = BIAS ? kLog2e : a.scale_log2;
    const float tau = (Lq == 1 || a.decode_pack) ? 0.f : (float)MFA_RESCALE_TAU;
    const float tau_c = tau / c;
    const float slope = a.alibi ? a.alibi[b * a.alibi_bstride + hq] : 0.f;
    // a key past the second 16 never carries weight when Lk <= 16: one PV step
    const bool two_steps = Lk > 16;

#pragma unroll
    for (int n = 0; n < NQ; ++n) {
        const int wq0 = q0 + (wave * NQ + n) * 32;  // this wavefront's n-th block
        if (wq0 >= Lq) break;
        // rows -> LDS -> B operands (row l32, k-slots 16*s + 8*half..); the
        // wave's own LDS operations complete in order
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
            const int ch = lane + 64 * i;
            *reinterpret_cast<u32x4_t*>(qo + (ch / CPR) * KST + (ch % CPR) * 8) = qn[i];
        }
        op_t qf[DS];
#pragma unroll
        for (int s = 0; s < DS; ++s) qf[s] = *reinterpret_cast<const op_t*>(qo + l32 * KST + 16 * s + 8 * half);
        if (n + 1 < NQ) load_q(n + 1);
        const int row = wq0 + l32;
        RowState rs[1];
        rs[0].center = row + dq;
        rs[0].lo = key_lo(a, rs[0].center);
        rs[0].hi = key_hi(a, rs[0].center, Lk);
        rs[0].slope = slope;
        row_reset(rs[0]);
        f32x16_t sacc[1];
#pragma unroll
        for (int s = 0; s < DS; ++s) sacc[0] = mfma16(kf[s], qf[s], s == 0 ? f32x16_t{} : sacc[0]);
        qb_transform<1, BIAS, true>(a, sacc, rs[0], 0, half);
        float alpha;
        (void)qb_update(rs[0], qb_max<1>(sacc), c, tau_c, alpha);  // from the empty state: O is still zero
        u32x4_t pw[1][2];
        qb_probs16<1, IS_BF16>(sacc, pw, rs[0].l, rs[0].mu, c);
        f32x16_t o[1][DB];
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            o[0][db] = mfma16(vf[db][0], __builtin_bit_cast(op_t, pw[0][0]), f32x16_t{});
            if (two_steps) o[0][db] = mfma16(vf[db][1], __builtin_bit_cast(op_t, pw[0][1]), o[0][db]);
        }
        if (a.out_f32) {  // the fp32 parity output: the common store
            store_out<1, DB, IS_BF16>(a, sv, o, rs, wq0, lane, c);
            continue;
        }
        // normalised 16-bit rows -> LDS (this lane: row l32, d = 32*db + 8*g +
        // 4*half..+3) -> row-contiguous global stores; the lse as elsewhere
        const float l = sum_halves(rs[0].l);
        const float inv = l > 0.f ? 1.f / l : 0.f;  // fully masked rows -> 0 (_kernel.py:85)
        if (sv.lse && half == 0 && row < Lq)
            sv.lse[row] = l > 0.f ? (rs[0].mu + __builtin_amdgcn_logf(l)) * kLn2 : -INFINITY;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float v0 = o[0][db][4 * g] * inv, v1 = o[0][db][4 * g + 1] * inv;
                const float v2 = o[0][db][4 * g + 2] * inv, v3 = o[0][db][4 * g + 3] * inv;
                u32x2_t w;
                if constexpr (IS_BF16) {
                    typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
                    w = __builtin_bit_cast(u32x2_t, bf16x4_t{(__bf16)v0, (__bf16)v1, (__bf16)v2, (__bf16)v3});
                } else {
                    typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4_t;
                    w = __builtin_bit_cast(u32x2_t, f16x4_t{(_Float16)v0, (_Float16)v1, (_Float16)v2, (_Float16)v3});
                }
                *reinterpret_cast<u32x2_t*>(qo + l32 * KST + 32 * db + 8 * g + 4 * half) = w;
            }
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
            const int ch = lane + 64 * i, orow = wq0 + ch / CPR, col = (ch % CPR) * 8;
            const u32x4_t w = *reinterpret_cast<const u32x4_t*>(qo + (ch / CPR) * KST + col);
            if (orow < Lq && col < D)
                store_stream(reinterpret_cast<u32x4_t*>(sv.o + ((int64_t)orow * a.os + col) * 2), w);
        }
    }
}

// ----------------------------------------------------------------------------
// fp32 kernel: same structure with v_mfma_f32_32x32x2_f32.  K-slot layout of
// the 32x32x2 MFMA: lane (half, x) supplies k = half, so QK^T step s uses
// d = s + half*DP/2 and PV step r uses the key held in accumulator register r.
template <int DP, int NKB, bool BIAS, bool PAGED>
__global__ void __launch_bounds__(kThreads) mfa_fwd32_kernel(KArgs a) {
    constexpr int QB = 1;
    constexpr int BM = kWaves * 32;
    constexpr int BN = NKB * 32;
    constexpr int DH = DP / 2;   // d values per half-wave
    constexpr int DB = DP / 32;
    constexpr int KST = DP + 4;  // K / Q row stride (floats)
    constexpr int VST = DP + 8;  // V row stride (floats): the half-waves read rows 4 apart
    constexpr int K_ELEMS = BN * KST;
    constexpr int V_ELEMS = BN * VST;
    constexpr int KV_ELEMS = 2 * (K_ELEMS + V_ELEMS);
    constexpr int Q_ELEMS = BM * KST;
    constexpr int SMEM = KV_ELEMS > Q_ELEMS ? KV_ELEMS : Q_ELEMS;
    constexpr int CPR = DP / 4;
    constexpr int KCH = (BN * CPR + kThreads - 1) / kThreads;

    __shared__ __attribute__((aligned(16))) float smem[SMEM];

    int b, hq, tile;
    if (!decode_tile(a, blockIdx.x, b, hq, tile)) return;
    const SeqView sv = seq_view<4>(a, b, hq);
    const int q0 = tile * BM;
    if (q0 >= sv.Lq) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int Lq = sv.Lq, Lk = sv.Lk, D = a.D;
    const int dq = Lk - Lq;

    // Q tile -> LDS (every chunk of this thread loaded before any is stored)
    {
        constexpr int QCH = (BM * CPR + kThreads - 1) / kThreads;  // chunks per thread
        u32x4_t val[QCH];
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
            const int c = tid + kThreads * i;
            const int row = c / CPR, col = (c % CPR) * 4;
            val[i] = u32x4_t{0, 0, 0, 0};
            if (c < BM * CPR && q0 + row < Lq && col < D)
                val[i] = *reinterpret_cast<const u32x4_t*>(sv.q + ((int64_t)(q0 + row) * a.qs + col) * 4);
        }
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
            const int c = tid + kThreads * i;
            if (QCH * kThreads == BM * CPR || c < BM * CPR)
                *reinterpret_cast<u32x4_t*>(smem + (c / CPR) * KST + (c % CPR) * 4) = val[i];
        }
    }
    __syncthreads();
    const int wq0 = q0 + wave * 32;
    float qf[DH];
#pragma unroll
    for (int s = 0; s < DH; s += 4) {
        const float4 t = *reinterpret_cast<const float4*>(smem + (wave * 32 + l32) * KST + half * DH + s);
        qf[s] = t.x;
        qf[s + 1] = t.y;
        qf[s + 2] = t.z;
        qf[s + 3] = t.w;
    }
    __syncthreads();

    RowState rs[QB];
    rs[0].center = wq0 + l32 + dq;
    rs[0].lo = key_lo(a, rs[0].center);
    rs[0].hi = key_hi(a, rs[0].center, Lk);
    rs[0].slope = a.alibi ? a.alibi[b * a.alibi_bstride + hq] : 0.f;
    row_reset(rs[0]);
    f32x16_t o[QB][DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[0][db][r] = 0.f;
    const float c = BIAS ? kLog2e : a.scale_log2;
    const float tau_c = (float)MFA_RESCALE_TAU / c;

    const int qlast = min(q0 + BM, Lq) - 1;
    const int klo = key_lo(a, q0 + dq);
    const int khi = key_hi(a, qlast + dq, Lk);
    const int jbeg = (klo / BN) * BN;
    const int nblk = khi >= klo ? (khi - jbeg) / BN + 1 : 0;
    const int wlast = min(wq0 + 32, Lq) - 1;
    const bool wave_live = wlast >= wq0;
    const int w_lo_first = key_lo(a, wq0 + dq), w_lo_last = key_lo(a, wlast + dq);
    const int w_hi_first = key_hi(a, wq0 + dq, Lk), w_hi_last = key_hi(a, wlast + dq, Lk);

    u32x4_t kreg[KCH], vreg[KCH];
    auto gload = [&](int j) {
        bool kok, vok;
        const int64_t kbo = kv_block_off<PAGED>(a, sv, j, Lk, a.kb, a.ks, kok);
        const int64_t vbo = kv_block_off<PAGED>(a, sv, j, Lk, a.vb, a.vs, vok);
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int cc = tid + kThreads * i;
            const int row = cc / CPR, col = (cc % CPR) * 4;
            const bool ok = (cc < BN * CPR) && (j + row < Lk) && (col < D) && kok && vok;
            u32x4_t kv = {0, 0, 0, 0}, vv = {0, 0, 0, 0};
            if (ok) {
                kv = *reinterpret_cast<const u32x4_t*>(sv.k + (kbo + (int64_t)row * a.ks + col) * 4);
                vv = *reinterpret_cast<const u32x4_t*>(sv.v + (vbo + (int64_t)row * a.vs + col) * 4);
            }
            kreg[i] = kv;
            vreg[i] = vv;
        }
    };
    auto swrite = [&](int buf) {
        float* kbuf = smem + buf * K_ELEMS;
        float* vbuf = smem + 2 * K_ELEMS + buf * V_ELEMS;
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int cc = tid + kThreads * i;
            if (cc < BN * CPR) {
                const int row = cc / CPR, col = (cc % CPR) * 4;
                *reinterpret_cast<u32x4_t*>(kbuf + row * KST + col) = kreg[i];
                *reinterpret_cast<u32x4_t*>(vbuf + row * VST + col) = vreg[i];
            }
        }
    };
    auto block = [&](auto masked_tag, const float* kbuf, const float* vbuf, int j) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        f32x16_t sacc[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
#pragma unroll
            for (int s = 0; s < DH; s += 4) {
                const float4 kf = *reinterpret_cast<const float4*>(kbuf + (32 * kb + l32) * KST + half * DH + s);
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, qf[s], sacc[kb], 0, 0, 0);
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, qf[s + 1], sacc[kb], 0, 0, 0);
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, qf[s + 2], sacc[kb], 0, 0, 0);
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, qf[s + 3], sacc[kb], 0, 0, 0);
            }
        }
        qb_transform<NKB, BIAS, MASKED, true>(a, sacc, rs[0], j, half);
        float alpha;
        if (qb_update(rs[0], qb_max<NKB>(sacc), c, tau_c, alpha)) scale_rows<DB>(o[0], alpha);
        qb_probs32<NKB>(sacc, rs[0].l, rs[0].mu, c);
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float vf = vbuf[(32 * kb + 4 * half + acc_row(r)) * VST + 32 * db + l32];
                    o[0][db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf, sacc[kb][r], o[0][db], 0, 0, 0);
                }
    };

    if (nblk > 0) {
        gload(jbeg);
        swrite(0);
    }
    for (int it = 0; it < nblk; ++it) {
        const int j = jbeg + it * BN;
        const int buf = it & 1;
        const bool more = it + 1 < nblk;
        if (more) gload(j + BN);
        __syncthreads();

        const bool skip = !wave_live || (j + BN - 1 < w_lo_first) || (j > w_hi_last);
        if (!skip) {
            const bool masked = !((j >= w_lo_last) && (j + BN - 1 <= w_hi_first));
            const float* kbuf = smem + buf * K_ELEMS;
            const float* vbuf = smem + 2 * K_ELEMS + buf * V_ELEMS;
            if (masked)
                block(std::true_type{}, kbuf, vbuf, j);
            else
                block(std::false_type{}, kbuf, vbuf, j);
        }
        if (more) swrite(buf ^ 1);
    }

    // fp32 output (out_f32 is implied for fp32 input)
    store_out<QB, DB, true>(a, sv, o, rs, wq0, lane, c);
    if constexpr (BIAS) {
        // the lse of the unshifted ALiBi scores (qb_transform's PRECISE form)
        if (a.alibi && sv.lse && half == 0) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const int qrow = wq0 + 32 * qb + l32;
                if (qrow < sv.Lq) sv.lse[qrow] -= rs[qb].slope * (float)row_dmin(rs[qb]);
            }
        }
    }
}

// ----------------------------------------------------------------------------
// host side

thread_local char g_err[512] = "";

int set_err(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

typedef void (*kernel_fn)(KArgs);

struct KernelCfg {
    kernel_fn fn;
    int rows;  // query rows per workgroup
    int keys;  // keys per K/V block
    int lds;   // LDS bytes
    const char* name;
    int threads = kThreads;  // threads per workgroup
};

template <int DP, int QB, int NKB, bool IS_BF16, bool BIAS, bool EXACT = false>
KernelCfg cfg16(const char* name, bool paged) {
    constexpr int BM = kWaves * QB * 32, BN = NKB * 32;
    constexpr int kv = 2 * (BN * (DP + 8) + BN * (DP + MFA_V_PAD)), qs = BM * (DP + 8);
    return KernelCfg{paged ? (kernel_fn)mfa_fwd16_kernel<DP, QB, NKB, IS_BF16, BIAS, true, EXACT>
                           : (kernel_fn)mfa_fwd16_kernel<DP, QB, NKB, IS_BF16, BIAS, false, EXACT>,
                     BM, BN, 2 * (kv > qs ? kv : qs), name};
}
// the exact-row kernel: one 32-row query block per wavefront (128-row tiles),
// 64-key blocks
template <bool IS_BF16, bool BIAS>
KernelCfg select16x(int dp, bool paged) {
    switch (dp) {
        case 32: return cfg16<32, 1, 2, IS_BF16, BIAS, true>(IS_BF16 ? "mfa_fwd16x<bf16,d32>" : "mfa_fwd16x<f16,d32>", paged);
        case 64: return cfg16<64, 1, 2, IS_BF16, BIAS, true>(IS_BF16 ? "mfa_fwd16x<bf16,d64>" : "mfa_fwd16x<f16,d64>", paged);
        case 96: return cfg16<96, 1, 2, IS_BF16, BIAS, true>(IS_BF16 ? "mfa_fwd16x<bf16,d96>" : "mfa_fwd16x<f16,d96>", paged);
        default: return cfg16<128, 1, 2, IS_BF16, BIAS, true>(IS_BF16 ? "mfa_fwd16x<bf16,d128>" : "mfa_fwd16x<f16,d128>", paged);
    }
}
template <int DP, int QB, int NKB, bool IS_BF16, bool BIAS, int NW = 8>
KernelCfg cfg16pp(const char* name) {
    constexpr int BM = NW * QB * 32, BN = NKB * 32;
    constexpr int kv = 2 * 3 * BN * DP, qs = BM * (DP + 8);  // three K and three V stages / Q staging
    return KernelCfg{mfa_fwd16_pp_kernel<DP, QB, NKB, IS_BF16, BIAS, NW>, BM, BN, 2 * (kv > qs ? kv : qs) + 16, name,
                     NW * 64};
}
template <int DP, bool IS_BF16, bool BIAS>
KernelCfg cfg16tk(const char* name) {
    constexpr int BM = kWaves * MFA_TK_BLOCKS * 32;
    return KernelCfg{mfa_fwd16_tk_kernel<DP, IS_BF16, BIAS>, BM, 32, 2 * 32 * (kWaves + 2) * (DP + 8), name};
}
template <bool IS_BF16, bool BIAS>
KernelCfg select16tk(int dp) {
    switch (dp) {
        case 32: return cfg16tk<32, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16tk<bf16,d32>" : "mfa_fwd16tk<f16,d32>");
        case 64: return cfg16tk<64, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16tk<bf16,d64>" : "mfa_fwd16tk<f16,d64>");
        case 96: return cfg16tk<96, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16tk<bf16,d96>" : "mfa_fwd16tk<f16,d96>");
        default: return cfg16tk<128, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16tk<bf16,d128>" : "mfa_fwd16tk<f16,d128>");
    }
}
template <int DP, int NKB, bool BIAS>
KernelCfg cfg32(const char* name, bool paged) {
    constexpr int BM = kWaves * 32, BN = NKB * 32;
    constexpr int kv = 2 * (BN * (DP + 4) + BN * (DP + 8)), qs = BM * (DP + 4);
    return KernelCfg{paged ? (kernel_fn)mfa_fwd32_kernel<DP, NKB, BIAS, true>
                           : (kernel_fn)mfa_fwd32_kernel<DP, NKB, BIAS, false>,
                     BM, BN, 4 * (kv > qs ? kv : qs), name};
}

// tile configuration per (dtype, padded head dim, bias)
// Tile shape per padded head dim: QB 32-query blocks per wavefront, NKB
// 32-key blocks per K/V block (overridable at build time for tuning sweeps).
#ifndef MFA_D32_TILE
#define MFA_D32_TILE 2, 2
#endif
#ifndef MFA_D64_TILE
#define MFA_D64_TILE 2, 2
#endif
#ifndef MFA_D96_TILE
#define MFA_D96_TILE 1, 2
#endif
#ifndef MFA_D128_TILE
#define MFA_D128_TILE 1, 2
#endif
#define MFA_STR2(...) #__VA_ARGS__
#define MFA_STR(...) MFA_STR2(__VA_ARGS__)

// bf16/fp16 calls use the ping-pong kernel (8 wavefronts) when its tiles fill
// the chip (make_plan decides): 512-row tiles (two 32-row query blocks per
// wavefront) or 256-row tiles (one) at head dims up to 64, 256-row tiles at
// head dim 128.  Head dim 96 has no ping-pong tiles.
#ifndef MFA_PINGPONG
#define MFA_PINGPONG 1
#endif
// ping-pong tiles pack the query heads of a K/V head (2, 4 or 8 of them)
#ifndef MFA_PP_HEAD_PACK
#define MFA_PP_HEAD_PACK 1
#endif
// ... and so do the 4-wavefront 16-bit tiles (2 or 4 heads)
#ifndef MFA_4W_HEAD_PACK
#define MFA_4W_HEAD_PACK 1
#endif
// paged K/V (block_table) runs on the 256-row and fp32 kernels only
template <bool IS_BF16, bool BIAS>
KernelCfg select16(int dp, bool fills_chip, bool paged, bool pp256) {
    if (MFA_PINGPONG && fills_chip && dp == 128)  // one 32-row query block per wavefront
        return cfg16pp<128, 1, 2, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16pp<bf16,d128,1,2>" : "mfa_fwd16pp<f16,d128,1,2>");
    if (MFA_PINGPONG && fills_chip && dp <= 64 && pp256) {  // one 32-row query block per wavefront
        if (dp == 32)
            return cfg16pp<32, 1, 2, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16pp<bf16,d32,1,2>" : "mfa_fwd16pp<f16,d32,1,2>");
        return cfg16pp<64, 1, 2, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16pp<bf16,d64,1,2>" : "mfa_fwd16pp<f16,d64,1,2>");
    }
    if constexpr (MFA_PP_NW16 && !BIAS) {  // four wavefronts per SIMD (with a bias they spill)
        if (MFA_PINGPONG && fills_chip && dp <= 64) {
            if (dp == 32)
                return cfg16pp<32, 1, 2, IS_BF16, BIAS, 16>(IS_BF16 ? "mfa_fwd16pp<bf16,d32,1,2,16w>" : "mfa_fwd16pp<f16,d32,1,2,16w>");
            return cfg16pp<64, 1, 2, IS_BF16, BIAS, 16>(IS_BF16 ? "mfa_fwd16pp<bf16,d64,1,2,16w>" : "mfa_fwd16pp<f16,d64,1,2,16w>");
        }
    }
    if (MFA_PINGPONG && fills_chip && dp <= 64) {
        if (dp == 32)
            return cfg16pp<32, 2, 2, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16pp<bf16,d32,2,2>" : "mfa_fwd16pp<f16,d32,2,2>");
        return cfg16pp<64, 2, 2, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16pp<bf16,d64,2,2>" : "mfa_fwd16pp<f16,d64,2,2>");
    }
    switch (dp) {
        case 32: return cfg16<32, MFA_D32_TILE, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16<bf16,d32," MFA_STR(MFA_D32_TILE) ">" : "mfa_fwd16<f16,d32," MFA_STR(MFA_D32_TILE) ">", paged);
        case 64:
            // with a bias two query blocks per wavefront exceed the register
            // budget and spill to scratch inside the loop (2.2-2.8x slower)
            if constexpr (BIAS)
                return cfg16<64, 1, 2, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16<bf16,d64,1, 2>" : "mfa_fwd16<f16,d64,1, 2>", paged);
            else
                return cfg16<64, MFA_D64_TILE, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16<bf16,d64," MFA_STR(MFA_D64_TILE) ">" : "mfa_fwd16<f16,d64," MFA_STR(MFA_D64_TILE) ">", paged);
        case 96: return cfg16<96, MFA_D96_TILE, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16<bf16,d96," MFA_STR(MFA_D96_TILE) ">" : "mfa_fwd16<f16,d96," MFA_STR(MFA_D96_TILE) ">", paged);
        default: return cfg16<128, MFA_D128_TILE, IS_BF16, BIAS>(IS_BF16 ? "mfa_fwd16<bf16,d128," MFA_STR(MFA_D128_TILE) ">" : "mfa_fwd16<f16,d128," MFA_STR(MFA_D128_TILE) ">", paged);
    }
}
template <bool BIAS>
KernelCfg select32(int dp, bool paged) {
    switch (dp) {
        case 32: return cfg32<32, 1, BIAS>("mfa_fwd32<f32,d32,q32,k32>", paged);
        case 64: return cfg32<64, 1, BIAS>("mfa_fwd32<f32,d64,q32,k32>", paged);
        case 96: return cfg32<96, 1, BIAS>("mfa_fwd32<f32,d96,q32,k32>", paged);
        default: return cfg32<128, 1, BIAS>("mfa_fwd32<f32,d128,q32,k32>", paged);
    }
}

struct Plan {
    KernelCfg cfg;
    KArgs args;
    int grid;
    bool empty;
    kernel_fn combine = nullptr;  // split-KV merge kernel
    int64_t ws_bytes = 0;         // split-KV workspace
    // second launch (after the first, before a split-KV merge): the exact-row
    // kernel on the single-row sequences of a varlen call that mixes them
    // with longer ones
    bool second = false;
    KernelCfg cfg2;
    KArgs args2;
    int grid2 = 0;
};

// Enqueue a plan's kernel launches (the split-KV merge aside).
void launch_plan(const Plan& plan, hipStream_t st) {
    hipLaunchKernelGGL(plan.cfg.fn, dim3(plan.grid), dim3(plan.cfg.threads), 0, st, plan.args);
    if (plan.second)
        hipLaunchKernelGGL(plan.cfg2.fn, dim3(plan.grid2), dim3(plan.cfg2.threads), 0, st, plan.args2);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Ping-pong tile height for dense causal / windowed calls, where tiles cost
// different amounts.  Each choice's time is estimated as max(heaviest tile,
// total work / CUs) -- what heaviest-first scheduling reaches -- in units of
// one 512-row x 64-key block; a 256-row x 64-key block costs 0.545 of one
// (the two tile heights' measured non-causal rates differ by 9%).  When the
// 512-row tiles all run at once the heaviest sets the time, and 256-row
// tiles, paired heavy with light on each CU, nearly halve it.
int64_t host_key_lo(const mfa_fwd_params* p, int64_t c) {
    return p->window_left >= 0 ? std::max<int64_t>(c - p->window_left, 0) : 0;
}
int64_t host_key_hi(const mfa_fwd_params* p, int64_t c) {
    int64_t hi = p->seqlen_k - 1;
    if (p->causal) hi = std::min<int64_t>(hi, c);
    if (p->window_right >= 0) hi = std::min<int64_t>(hi, c + p->window_right);
    return hi;
}
double tile_makespan(const mfa_fwd_params* p, int rows, double block_cost, int cus) {
    const int64_t dq = (int64_t)p->seqlen_k - p->seqlen_q;
    const int64_t T = (p->seqlen_q + rows - 1) / rows;
    int64_t heaviest = 0, total = 0;
    for (int64_t t = 0; t < T; ++t) {
        const int64_t r0 = t * rows, r1 = std::min<int64_t>(r0 + rows, p->seqlen_q) - 1;
        const int64_t lo = host_key_lo(p, r0 + dq), hi = host_key_hi(p, r1 + dq);
        const int64_t n = hi >= lo ? hi / 64 - lo / 64 + 1 : 0;
        heaviest = std::max(heaviest, n);
        total += n;
    }
    const double units = (double)p->batch * p->heads_q;
    return std::max((double)heaviest, units * (double)total / cus) * block_cost;
}
bool prefer_pp256(const mfa_fwd_params* p, int cus) {
    if (p->cu_seqlens_q || (!p->causal && p->window_left < 0 && p->window_right < 0)) return false;
    if (p->seqlen_q > (1 << 20)) return false;  // (bounds the estimate's loop; long rows balance anyway)
    return tile_makespan(p, 256, 0.545, cus) < 0.9 * tile_makespan(p, 512, 1.0, cus);
}

// ---- Chip geometry: compute units and XCDs of the device a call runs on,
// looked up once per device (hipDeviceGetAttribute with the device current)
// and kept.  The tile choices compare grids against the CU count, and the
// grouped schedule deals workgroups over the XCDs.  MI355X: 256 CUs in 8
// XCDs, also the defaults when no device is visible (planning-only calls on a
// host without a GPU).  MTLFLASHATTN_CHIP_CUS / MTLFLASHATTN_CHIP_XCDS
// override the values (tuning and tests).
struct ChipGeom {
    int cus = 256;
    int xcds = 8;
};
constexpr int kMaxGeomDevices = 256;
std::mutex g_geom_mu;
ChipGeom g_geom[kMaxGeomDevices];
bool g_geom_known[kMaxGeomDevices];

int env_positive(const char* name) {
    const char* v = getenv(name);
    if (!v || !*v) return 0;
    const long x = strtol(v, nullptr, 10);
    return x > 0 && x < (1 << 20) ? (int)x : 0;
}

ChipGeom chip_geometry(int dev) {
    ChipGeom g;
    if (dev < 0 || dev >= kMaxGeomDevices) return g;
    std::lock_guard<std::mutex> lock(g_geom_mu);
    if (!g_geom_known[dev]) {
        int cur = -1, v = 0;
        if (hipGetDevice(&cur) == hipSuccess) {
            const bool switch_dev = cur != dev && hipSetDevice(dev) == hipSuccess;
            if ((switch_dev || cur == dev) &&
                hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
                g.cus = v;
            if ((switch_dev || cur == dev) &&
                hipDeviceGetAttribute(&v, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess && v > 0)
                g.xcds = v;
            if (switch_dev) (void)hipSetDevice(cur);
        }
        (void)hipGetLastError();  // a failed query leaves no sticky error for the caller
        if (const int e = env_positive("MTLFLASHATTN_CHIP_CUS")) g.cus = e;
        if (const int e = env_positive("MTLFLASHATTN_CHIP_XCDS")) g.xcds = e;
        g_geom[dev] = g;
        g_geom_known[dev] = true;
    }
    return g_geom[dev];
}
// geometry of the device `st` belongs to (the current device for the null stream)
ChipGeom chip_geometry_of(hipStream_t st) {
    int dev = -1;
    const hipError_t e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        dev = 0;
    }
    return chip_geometry(dev);
}
ChipGeom chip_geometry_current() { return chip_geometry_of(nullptr); }

int make_plan(const mfa_fwd_params* p, Plan* plan, const ChipGeom& geom, int split_keys = 0) {
    if (!p) return set_err(MFA_ERR_INVALID, "mfa_fwd: params is NULL");
    // Single-row grouped-query decode: the R query heads of a K/V head become
    // the R rows of one sequence (the same q/o memory through other strides),
    // so one workgroup reads each K/V head once for all of them.  Exact for
    // rows whose valid keys do not depend on their position -- no window, no
    // ALiBi; causal with one query row admits every key -- and, with the
    // per-row rescales of such rows, bit-identical to the unpacked call.
    // Varlen calls whose longest query is one row pack the same way (a
    // sequence's rows are its one token's query heads); there the lse rows
    // of one token would not be contiguous, so only without an lse output.
    const int64_t tok_qs = p->q_seq_stride, tok_os = p->o_seq_stride;  // token strides (varlen starts)
    mfa_fwd_params packed;
    bool pack = false;
    const bool lse_ok = p->cu_seqlens_q ? !p->softmax_lse : (!p->softmax_lse || p->lse_head_stride == 1);
    if (p->dtype_in != MFA_DTYPE_F32 && p->seqlen_q == 1 && p->heads_kv > 0 && p->heads_q > p->heads_kv &&
        p->heads_q % p->heads_kv == 0 && p->window_left < 0 && p->window_right < 0 && !p->alibi_slopes && lse_ok) {
        const int R = p->heads_q / p->heads_kv;
        packed = *p;
        packed.seqlen_q = R;
        packed.heads_q = p->heads_kv;
        packed.q_seq_stride = p->q_head_stride;
        packed.q_head_stride = p->q_head_stride * R;
        packed.o_seq_stride = p->o_head_stride;
        packed.o_head_stride = p->o_head_stride * R;
        packed.causal = 0;
        if (p->softmax_lse) packed.lse_head_stride = R;
        p = &packed;
        pack = true;
    }
    const int din = p->dtype_in, dout = p->dtype_out;
    if (din != MFA_DTYPE_F16 && din != MFA_DTYPE_BF16 && din != MFA_DTYPE_F32)
        return set_err(MFA_ERR_INVALID, "mfa_fwd: unknown dtype_in %d", din);
    if (dout != din && dout != MFA_DTYPE_F32)
        return set_err(MFA_ERR_INVALID, "mfa_fwd: dtype_out %d must equal dtype_in %d or be fp32", dout, din);
    const int D = p->head_dim;
    if (D <= 0 || D > MFA_MAX_HEAD_DIM)
        return set_err(MFA_ERR_UNSUPPORTED, "mfa_fwd: head_dim %d outside [1, %d]", D, MFA_MAX_HEAD_DIM);
    if (D % 8 != 0)
        return set_err(MFA_ERR_UNSUPPORTED, "mfa_fwd: head_dim %d is not a multiple of 8 (pad it)", D);
    if (p->batch < 0 || p->seqlen_q < 0 || p->seqlen_k < 0)
        return set_err(MFA_ERR_INVALID, "mfa_fwd: negative batch/seqlen (%d, %d, %d)", p->batch, p->seqlen_q,
                       p->seqlen_k);
    if (p->heads_q <= 0 || p->heads_kv <= 0 || p->heads_q % p->heads_kv != 0)
        return set_err(MFA_ERR_INVALID, "mfa_fwd: num_heads_kv (%d) must divide num_heads_q (%d)", p->heads_kv,
                       p->heads_q);
    if (!(p->softcap >= 0.f)) return set_err(MFA_ERR_INVALID, "mfa_fwd: softcap must be >= 0");
    if (p->window_left < -1 || p->window_right < -1)
        return set_err(MFA_ERR_INVALID, "mfa_fwd: window bounds must be >= -1");
    if ((p->cu_seqlens_q == nullptr) != (p->cu_seqlens_k == nullptr))
        return set_err(MFA_ERR_INVALID, "mfa_fwd: cu_seqlens_q and cu_seqlens_k must both be set or both NULL");
    if (p->block_table) {
        // every key block lies inside one page: block sizes (32..128 keys) and
        // split chunks divide the page size
        if (p->page_block_size <= 0 || p->page_block_size % 256 != 0)
            return set_err(MFA_ERR_INVALID, "mfa_fwd: page_block_size %d must be a positive multiple of 256",
                           p->page_block_size);
        if (p->num_pages <= 0) return set_err(MFA_ERR_INVALID, "mfa_fwd: num_pages must be > 0 with a block_table");
        if (p->block_table_batch_stride < 0)
            return set_err(MFA_ERR_INVALID, "mfa_fwd: block_table_batch_stride must be >= 0");
        if (split_keys % 256 != 0)
            return set_err(MFA_ERR_INVALID, "mfa_fwd_splitkv: split_keys %d must be a multiple of 256 with a block_table",
                           split_keys);
    }
    if (p->softmax_lse && (p->lse_batch_stride < 0 || p->lse_head_stride < 0))
        return set_err(MFA_ERR_INVALID, "mfa_fwd: lse strides must be >= 0");

    plan->empty = (p->batch == 0 || p->seqlen_q == 0);
    const int es = din == MFA_DTYPE_F32 ? 4 : 2;
    const int oes = dout == MFA_DTYPE_F32 ? 4 : 2;
    if (!plan->empty) {
        if (!p->q || !p->k || !p->v || !p->o) return set_err(MFA_ERR_INVALID, "mfa_fwd: NULL tensor pointer");
        if (!aligned16(p->q) || !aligned16(p->k) || !aligned16(p->v) || !aligned16(p->o))
            return set_err(MFA_ERR_INVALID, "mfa_fwd: q/k/v/o must be 16-byte aligned");
        const int64_t in_al = 16 / es;  // elements per 16 bytes
        const int64_t s_in[9] = {p->q_batch_stride, p->q_seq_stride, p->q_head_stride,
                                 p->k_batch_stride, p->k_seq_stride, p->k_head_stride,
                                 p->v_batch_stride, p->v_seq_stride, p->v_head_stride};
        for (int i = 0; i < 9; ++i)
            if (s_in[i] % in_al != 0)
                return set_err(MFA_ERR_INVALID, "mfa_fwd: q/k/v strides must be multiples of %lld elements",
                               (long long)in_al);
        // O leaves the 16-bit kernels in row-contiguous 16-byte pieces (and a
        // packed grouped-query decode uses the head stride as its row stride),
        // so every o stride is a multiple of 16 bytes, as for q/k/v
        const int64_t out_al = 16 / oes;
        if (p->o_batch_stride % out_al || p->o_seq_stride % out_al || p->o_head_stride % out_al)
            return set_err(MFA_ERR_INVALID, "mfa_fwd: o strides must be multiples of %lld elements (16 bytes)",
                           (long long)out_al);
        if (p->alibi_slopes && !(p->alibi_batch_stride == 0 || p->alibi_batch_stride == p->heads_q))
            return set_err(MFA_ERR_INVALID, "mfa_fwd: alibi_batch_stride must be 0 or heads_q");
    }

    // K/V blocks are addressed with 32-bit byte offsets from the block start
    const int64_t kv_span = (int64_t)63 * (p->k_seq_stride > p->v_seq_stride ? p->k_seq_stride : p->v_seq_stride);
    if (p->k_seq_stride < 0 || p->v_seq_stride < 0 || (kv_span + D) * es >= ((int64_t)1 << 31))
        return set_err(MFA_ERR_INVALID, "mfa_fwd: k/v sequence strides must be >= 0 and span < 2 GiB per 64 rows");

    const int dp = D <= 32 ? 32 : D <= 64 ? 64 : D <= 96 ? 96 : 128;
    const bool bias = p->softcap > 0.f || p->alibi_slopes != nullptr || !(p->scale > 0.f);
    // the 512-row ping-pong tiles are used when they still give every CU a
    // workgroup (256 CUs on MI355X)
    if (p->tile_hint < MFA_TILE_AUTO || p->tile_hint > MFA_TILE_PINGPONG256)
        return set_err(MFA_ERR_INVALID, "mfa_fwd: unknown tile_hint %d", p->tile_hint);
    const bool pp_hint = p->tile_hint == MFA_TILE_PINGPONG || p->tile_hint == MFA_TILE_PINGPONG256;
    if (pp_hint && (din == MFA_DTYPE_F32 || dp == 96))
        return set_err(MFA_ERR_UNSUPPORTED,
                       "mfa_fwd: ping-pong tiles need bf16/fp16 and head_dim <= 64 or 97..128");
    // Auto: ping-pong tiles (512 rows at head dims <= 64, 256 at 128) when
    // they fill the chip (one workgroup per CU) and leave at most 25% more
    // rows empty than the 4-wavefront kernel's tiles (256 / 128 rows) do:
    // short or single-row queries run faster on the 4-wavefront kernel.
    const int64_t rows512 = (int64_t)((p->seqlen_q + 511) / 512) * 512;
    const int64_t rows256 = (int64_t)((p->seqlen_q + 255) / 256) * 256;
    const int64_t units = (int64_t)p->batch * p->heads_q;
    bool fills_chip = pp_hint;
    if (p->tile_hint == MFA_TILE_AUTO) {
        if (dp == 128) {
            // Rows long enough: >= 2 tiles per head, 8 when causal (bf16,
            // ping-pong vs 4-wavefront, one box: non-causal B=64 L=256 64 vs
            // 61 us, B=32 L=512 88 vs 93, B=4 L=768 28 vs 32, B=16 L=1024 143
            // vs 157; causal B=16 L=1024 113 vs 111, B=16 L=1536 221 vs 219,
            // B=8 L=2048 166 vs 176, B=4 L=3072 177 vs 180).  All 8 wavefronts of a ping-pong workgroup walk
            // the key range of all its 256 rows, so a sliding window must be
            // wide against that: windows of >= 1536 keys (512 on packed
            // grouped-query tiles, below) run faster there (L=8192
            // (1024,1024) 145 vs 154 us, (4096,0) causal 234 vs 241, L=32768
            // (2048,0) causal 610 vs 634), narrower ones slower ((256,256)
            // 67 vs 61, (512,0) causal 67 vs 61).  A soft-cap /
            // ALiBi transform under a window stays on the 4-wavefront kernel
            // (L=32768 H=16 causal (2048,0) with soft-cap 30 and ALiBi: 832 vs
            // 791 us).  Varlen calls give only the longest sequence, and short
            // sequences waste half-empty 256-row tiles: the thresholds rise to
            // 5 tiles non-causal and 16 causal (H=16: 64 lengths in [128,
            // 1024] 338 vs 304 us, 32 in [256, 1280] 273 vs 283, 32 in [128,
            // 2048] 380 vs 373, 16 in [512, 1536] 175 vs 184; causal 16 in
            // [512, 1536] 129 vs 118, 8 in [1024, 4096] 298 vs 301).
            // A grouped-query call with 2, 4 or 8 query heads per K/V head
            // packs them into each tile (256 / R positions per ping-pong
            // tile): there rows go to the ping-pong tiles from 512 positions
            // when dense and non-causal, 1024 when varlen and non-causal and
            // 1280 when causal (bf16 Hq=32 Hkv=8, 4-wavefront vs ping-pong,
            // one box: non-causal B=32 L=512 181 vs 172 us, B=16 L=1024 317
            // vs 286; causal B=32 L=512 135 vs 143, B=16 L=1024 200 vs 199,
            // B=12 L=1536 295 vs 275; varlen 64 lengths in [64, 1024] 480 vs
            // 474 and causal 313 vs 320, 32 in [128, 1536] 700 vs 649 and
            // 420 vs 411).  All were 2048 before the ping-pong tiles got
            // cheaper (measured at Hq=32 Hkv=8
            // D=128 on packed tiles, ping-pong vs 4-wavefront: config 4's 8
            // varlen lengths in [863, 3501] causal 474 vs 516 us, non-causal
            // 802 vs 868; 16 lengths in [256, 4096] 919 vs 997 and 1610 vs
            // 1770; 32 in [128, 2048] 623 vs 624 and 991 vs 1065; 64 in [64,
            // 1024] 389 vs 344 and 521 vs 496; B=4 L=2048 causal 162 vs 171).
            const int64_t Rq = p->heads_kv > 0 ? p->heads_q / p->heads_kv : 1;
            const bool packs = MFA_PP_HEAD_PACK && (Rq == 2 || Rq == 4 || Rq == 8);
            const int64_t pos_pp = packs ? 256 / Rq : 256;  // positions per ping-pong tile
            const int64_t pos_4w = MFA_4W_HEAD_PACK && (Rq == 2 || Rq == 4) ? 128 / Rq : 128;
            const int64_t rows_pp = (p->seqlen_q + pos_pp - 1) / pos_pp * pos_pp;
            const int64_t rows_4w = (p->seqlen_q + pos_4w - 1) / pos_4w * pos_4w;
            const int64_t units_pp = packs ? (int64_t)p->batch * p->heads_kv : units;
            const int64_t t256 = rows_pp / pos_pp;
            const int64_t inf = INT64_MAX / 4;
            const int64_t left = p->window_left >= 0 ? p->window_left : inf;
            const int64_t right = p->causal ? 0 : p->window_right >= 0 ? p->window_right : inf;
            const bool windowed = p->window_left >= 0 || p->window_right >= 0;
            const int64_t min_pos = p->causal ? 1280 : p->cu_seqlens_q ? 1024 : 512;
            const int64_t min_tiles = packs              ? (min_pos + pos_pp - 1) / pos_pp
                                      : p->cu_seqlens_q ? (p->causal ? 16 : 5)
                                                        : (p->causal ? 8 : 2);
            // Windows: re-measured on the current tiles (bf16, 4-wavefront vs
            // ping-pong): unpacked L=8192 H=16 (512,511) 90.8 vs 90.4 us,
            // (768,767) 122 vs 118, causal (1024,0) 89.3 vs 90.0, (1536,0)
            // 119 vs 116; packed B=4 L=4096 Hq=32 Hkv=8 (256,256) 193 vs
            // 184, (512,511) 310 vs 284, causal (1024,0) 297 vs 276.
            const int64_t min_window = packs ? 512 : 1536;
            fills_chip = units_pp * t256 >= geom.cus && 4 * rows_pp <= 5 * rows_4w && t256 >= min_tiles &&
                         (!windowed || (!bias && left + right + 1 >= min_window));
        } else
            fills_chip = units * (rows512 / 512) >= geom.cus && 4 * rows512 <= 5 * rows256;
    }
    bool pp256 = p->tile_hint == MFA_TILE_PINGPONG256;
    if (split_keys != 0) {
        // split-KV runs on the 4-wavefront kernel (bf16/fp16)
        if (split_keys < 0 || split_keys % 64 != 0)
            return set_err(MFA_ERR_INVALID, "mfa_fwd_splitkv: split_keys %d must be a positive multiple of 64",
                           split_keys);
        if (din == MFA_DTYPE_F32) return set_err(MFA_ERR_UNSUPPORTED, "mfa_fwd_splitkv: fp32 has no split-KV path");
        if (pp_hint)
            return set_err(MFA_ERR_UNSUPPORTED, "mfa_fwd_splitkv: split-KV uses the 256-row tiles");
        fills_chip = false;
    }
    const bool paged = p->block_table != nullptr;
    if (paged) {
        if (pp_hint)
            return set_err(MFA_ERR_UNSUPPORTED, "mfa_fwd: ping-pong tiles do not take a block_table");
        fills_chip = false;
    }
    // Dense calls (no window, no bias) of rows >= 1024 whose 512-row tiles do
    // not fill the chip but whose 256-row ping-pong tiles do: those tiles (measured 15-25%
    // faster than the 4-wavefront kernel at D=64: causal B=1 L=4096 H=16 101
    // -> 80 us, B=1 L=8192 H=8 187 -> 146; non-causal B=1 L=4096 H=16 100 ->
    // 83, B=1 L=8192 H=8 188 -> 156).
    // Shorter rows (2-3 tiles of 256) take those tiles too when they make
    // 3/4 to one round of workgroups (bf16 H=8, 4-wavefront vs ping-pong:
    // D=64 B=12 L=512 18.2 vs 16.7 us, B=16 L=512 18.8 vs 17.3, B=10 L=768
    // 24.0 vs 21.9, causal B=16 L=512 21.3 vs 18.4; D=32 B=16 L=512 causal
    // 17.7 vs 16.1; just past one round they lose: D=64 B=18 L=512 25.1 vs
    // 30.4, B=11 L=768 33.5 vs 39.6).
    const int64_t t256 = rows256 / 256, n256 = units * t256;
    const bool one_round = t256 >= 2 && 4 * n256 >= 3 * (int64_t)geom.cus && n256 <= geom.cus &&
                           4 * rows256 <= 5 * (int64_t)p->seqlen_q;
    if (p->tile_hint == MFA_TILE_AUTO && !fills_chip && !paged && split_keys == 0 && dp <= 64 &&
        din != MFA_DTYPE_F32 && !bias && !p->cu_seqlens_q && p->window_left < 0 && p->window_right < 0 &&
        ((n256 >= geom.cus && t256 >= 4) || one_round)) {
        // (rows of >= 4 tiles over more rounds: shorter rows, e.g. B=64
        // L=256 H=16, run 40 vs 50 us on the 4-wavefront kernel)
        fills_chip = true;
        pp256 = true;
    } else if (p->tile_hint == MFA_TILE_AUTO && fills_chip && dp <= 64 && din != MFA_DTYPE_F32) {
        // Windowed calls, causal calls with a soft-cap / ALiBi transform and
        // varlen calls run faster on the 4-wavefront kernel (measured at
        // L=8192 H=16 D=64: window (2048,0) 99 vs 106 us, (256,256) 45 vs
        // 55, causal + soft-cap 261 vs 305; 8 varlen lengths in [863, 3501]
        // at D=64 Hq=32 Hkv=8: causal 306 vs 398 us, non-causal 512 vs 556): a
        // ping-pong workgroup's waves share one K/V stream, so rows whose
        // window ends early wait through the rest of it, and 512-row tiles
        // leave much of a short sequence's last tile empty.
        // Causal calls whose 512-row tiles are few per head (<= 8) and take
        // more than one round of workgroups go there as well (measured:
        // B=8 L=1024 Hq=32 68 vs 97 us, B=2 L=4096 Hq=32 Hkv=8 172 vs 190;
        // with one round, or longer rows, the ping-pong tiles win: L=4096
        // H=32 100 vs 117, B=2 L=8192 H=16 327 vs 345).
        // Rows of one 512-row tile per head go there too: non-causal (bf16
        // H=16 L=512, 4-wavefront vs ping-pong: B=32 D=64 50.2 vs 52.4 us,
        // B=64 D=64 96.7 vs 101.7, B=32 D=32 38.5 vs 42.1; at L=1024 the
        // ping-pong tiles win, B=16 D=64 83.5 vs 87.1), and causal ones in
        // a single round of 512-row tiles, whose 256-row tiles would take
        // two (B=32 L=512 H=8 D=64 23.5 vs 31.1 us).
        const bool windowed = p->window_left >= 0 || p->window_right >= 0;
        const int64_t t512 = rows512 / 512;
        if (windowed || (p->causal && bias) || p->cu_seqlens_q)
            fills_chip = false;
        else if (p->causal && t512 <= 8 && (units * t512 > geom.cus || t512 == 1))
            fills_chip = false;
        else if (!p->causal && t512 < 2)
            fills_chip = false;
        else
            pp256 = prefer_pp256(p, geom.cus);
    }
    // Exact rows: a 16-bit call whose every sequence has one query row, or a
    // packed grouped-query decode, runs the exact-row kernel (two-term
    // probabilities, per-row rescales), whatever the tile hint.  A varlen
    // call that may mix single-row sequences with longer ones runs its kernel
    // on the longer ones and the exact-row kernel on the single-row ones
    // (a second launch, planned below), so each sequence's rows are those of
    // its own dense call.
    const bool exact_call = din != MFA_DTYPE_F32 && (pack || p->seqlen_q == 1);
    const bool mixed_rows =
        din != MFA_DTYPE_F32 && !exact_call && p->cu_seqlens_q != nullptr && !p->varlen_no_single_rows;
    // At most 32 keys per sequence under many query rows (cross-attention to
    // a short conditioning sequence): the tiny-key kernel, which keeps the
    // keys in registers and streams the query rows (measured at bf16 D=128
    // Lq=26136 Lk=5 H=16: see the design notes)
    const bool tiny_keys = MFA_TK && p->tile_hint == MFA_TILE_AUTO && din != MFA_DTYPE_F32 && !paged &&
                           !exact_call && split_keys == 0 && p->seqlen_k <= 32 && p->seqlen_q >= MFA_TK_MIN_ROWS;
    auto exact_cfg = [&]() {
        if (din == MFA_DTYPE_BF16) return bias ? select16x<true, true>(dp, paged) : select16x<true, false>(dp, paged);
        return bias ? select16x<false, true>(dp, paged) : select16x<false, false>(dp, paged);
    };
    if (din == MFA_DTYPE_F32)
        plan->cfg = bias ? select32<true>(dp, paged) : select32<false>(dp, paged);
    else if (exact_call)
        plan->cfg = exact_cfg();
    else if (tiny_keys && din == MFA_DTYPE_BF16)
        plan->cfg = bias ? select16tk<true, true>(dp) : select16tk<true, false>(dp);
    else if (tiny_keys)
        plan->cfg = bias ? select16tk<false, true>(dp) : select16tk<false, false>(dp);
    else if (din == MFA_DTYPE_BF16)
        plan->cfg = bias ? select16<true, true>(dp, fills_chip, paged, pp256)
                         : select16<true, false>(dp, fills_chip, paged, pp256);
    else
        plan->cfg = bias ? select16<false, true>(dp, fills_chip, paged, pp256)
                         : select16<false, false>(dp, fills_chip, paged, pp256);

    KArgs& a = plan->args;
    memset(&a, 0, sizeof(a));
    a.q = static_cast<const char*>(p->q);
    a.k = static_cast<const char*>(p->k);
    a.v = static_cast<const char*>(p->v);
    a.o = static_cast<char*>(p->o);
    a.qb = p->q_batch_stride; a.qs = p->q_seq_stride; a.qh = p->q_head_stride;
    a.kb = p->k_batch_stride; a.ks = p->k_seq_stride; a.kh = p->k_head_stride;
    a.vb = p->v_batch_stride; a.vs = p->v_seq_stride; a.vh = p->v_head_stride;
    a.ob = p->o_batch_stride; a.os = p->o_seq_stride; a.oh = p->o_head_stride;
    a.cu_q = p->cu_seqlens_q;
    a.cu_k = p->cu_seqlens_k;
    a.alibi = p->alibi_slopes;
    a.alibi_bstride = p->alibi_batch_stride;
    a.B = p->batch; a.Hq = p->heads_q; a.Hkv = p->heads_kv;
    a.Lq = p->seqlen_q; a.Lk = p->seqlen_k; a.D = D;
    a.scale = p->scale;
    a.scale_log2 = p->scale * kLog2e;
    a.softcap = p->softcap;
    a.softcap_k = p->softcap > 0.f ? 2.f * kLog2e / p->softcap : 0.f;
    a.softcap_sk = p->scale * a.softcap_k;
    // clamp windows so center +/- window cannot overflow int32
    const int64_t wmax = (int64_t)p->seqlen_q + (int64_t)p->seqlen_k + 1;
    a.wl = p->window_left < 0 ? -1 : (int32_t)(p->window_left > wmax ? wmax : p->window_left);
    a.wr = p->window_right < 0 ? -1 : (int32_t)(p->window_right > wmax ? wmax : p->window_right);
    a.causal = p->causal ? 1 : 0;
    a.decode_pack = pack ? 1 : 0;
    a.qts = tok_qs;
    a.ots = tok_os;
    a.pack_r = (pack && p->cu_seqlens_q) ? p->seqlen_q : 1;  // packed varlen: R rows per query token
    a.single_rows = mixed_rows ? 1 : 0;
    a.out_f32 = dout == MFA_DTYPE_F32 ? 1 : 0;
    a.lse = p->softmax_lse;
    a.lse_b = p->lse_batch_stride;
    a.lse_h = p->lse_head_stride;
    if (p->block_table) {
        // j / page for 0 <= j < 2^31 as umulhi(j, m) >> s (round-up method:
        // l = ceil(log2 page), m = ceil(2^(31+l) / page) < 2^32, s = l - 1)
        const uint32_t d = (uint32_t)p->page_block_size;
        int l = 0;
        while ((1u << l) < d) ++l;
        const unsigned __int128 one = 1;
        a.page_m = (uint32_t)(((one << (31 + l)) + d - 1) / d);
        a.page_s = l - 1;
        a.page = p->page_block_size;
        a.npages = p->num_pages;
        a.bt = p->block_table;
        a.bt_b = p->block_table_batch_stride;
    } else {
        a.page_m = 0;  // one page: j / page = 0, row = j
        a.page_s = 0;
        a.page = 0;
        a.npages = 1;
        a.bt = nullptr;
        a.bt_b = 0;
    }

    // Ping-pong tiles of a grouped-query call with 2, 4 or 8 query heads per
    // K/V head pack those heads into one tile (KArgs.hpack): each head takes
    // 1/R of the tile's rows at the same positions, so a tile streams its K/V
    // once for R heads, and a causal tile spans 1/R of the positions (fewer
    // partly masked diagonal blocks).  Rows of one wavefront are still 32
    // consecutive positions of one head aligned to 32, so every row's
    // arithmetic equals the unpacked call's (grouped-query heads equal
    // repeated K/V heads bit for bit).
    a.hpack = 1;
    a.qh1 = a.qh;
    a.oh1 = a.oh;
    a.lse_h1 = a.lse_h;
    const int R = p->heads_q / p->heads_kv;
    // The 4-wavefront 16-bit kernel packs 2 or 4 heads the same way (one or
    // two wavefronts per head), except for split-KV and paged calls.
    const bool pack_pp = MFA_PP_HEAD_PACK && plan->cfg.threads == 8 * 64 && (R == 2 || R == 4 || R == 8);
    const bool pack_4w = MFA_4W_HEAD_PACK && din != MFA_DTYPE_F32 && !exact_call && !tiny_keys && !paged &&
                         split_keys == 0 && plan->cfg.threads == kThreads && (R == 2 || R == 4);
    if (pack_pp || pack_4w) {
        a.hpack = R;
        a.Hq = p->heads_kv;
        a.qh = p->q_head_stride * R;
        a.oh = p->o_head_stride * R;
        a.lse_h = p->lse_head_stride * R;
    }
    const int rows = plan->cfg.rows / a.hpack;  // positions per tile
    a.T = (p->seqlen_q + rows - 1) / rows;
    // (bounded before the int32 product below is formed)
    if ((int64_t)p->batch * p->heads_q * a.T > 0x7fffffffLL / 2)
        return set_err(MFA_ERR_INVALID, "mfa_fwd: problem too large");
    a.U = p->batch * a.Hq;
    const int64_t G = (int64_t)p->batch * p->heads_kv;
    const int X = geom.xcds;
    int xshift = 0;
    while ((1 << xshift) < X) ++xshift;
    if (G > 0 && (1 << xshift) == X && G % X == 0) {  // (a power-of-two XCD count dividing the groups)
        a.grouped = 1;
        a.xcd_shift = xshift;
        a.tile_major = (p->causal || p->window_left >= 0 || p->window_right >= 0) ? 1 : 0;
        // Head-packed varlen tiles run unit-major: a packed tile reads its K/V
        // once for its R heads, so the L2 reuse that tile-major order gets
        // from the R heads of one (sequence, K/V head) running side by side is
        // gone, and tiles of sequences of different lengths interleaved on an
        // XCD evict each other's K/V (config 4: 644 vs 494 us on the
        // 4-wavefront tiles, 617 vs 469 on the ping-pong ones).  Dense calls
        // keep tile-major order (B=4 L=2048 Hq=32 Hkv=8 causal 169 vs 173 us).
        if (a.hpack > 1 && p->cu_seqlens_q) a.tile_major = 0;
        a.upx = (int32_t)(G / X) * (a.Hq / p->heads_kv);
        plan->grid = X * a.upx * a.T;
    } else {
        a.grouped = 0;
        a.upx = 0;
        plan->grid = a.U * a.T;
    }
    if ((int64_t)a.U * a.T > 0x7fffffffLL / 2) return set_err(MFA_ERR_INVALID, "mfa_fwd: problem too large");
    a.nsplit = 1;
    if (split_keys != 0) {
        const int ns = (p->seqlen_k + split_keys - 1) / split_keys;
        if (ns > kMaxSplits)
            return set_err(MFA_ERR_INVALID, "mfa_fwd_splitkv: %d chunks of %d keys exceed %d; use larger chunks", ns,
                           split_keys, kMaxSplits);
        a.nsplit = ns > 1 ? ns : 1;
        a.split_keys = split_keys;
        a.ws_ld = dp;
        if ((int64_t)a.U * a.T * a.nsplit > 0x7fffffffLL / 2 ||
            (int64_t)a.nsplit * a.U * p->seqlen_q > 0x7fffffffLL)  // (the merge grid: one workgroup per row)
            return set_err(MFA_ERR_INVALID, "mfa_fwd_splitkv: too many splits");
        a.T *= a.nsplit;
        plan->grid *= a.nsplit;
        const int64_t rows = (int64_t)a.nsplit * a.U * p->seqlen_q;
        plan->ws_bytes = rows * dp * 4 + ((rows * 4 + 255) / 256) * 256;
        plan->combine = din == MFA_DTYPE_BF16 ? (kernel_fn)mfa_combine_kernel<true> : (kernel_fn)mfa_combine_kernel<false>;
    }
    if (plan->grid == 0) plan->empty = true;
    plan->second = false;
    if (mixed_rows && !plan->empty) {
        // the exact-row kernel over one query tile (times the split chunks)
        // of every (sequence, head); it computes the single-row sequences only
        plan->second = true;
        plan->cfg2 = exact_cfg();
        KArgs& a2 = plan->args2;
        a2 = a;
        a2.single_rows = 2;
        // (one head per unit: undo a head-packed main launch's strides)
        a2.hpack = 1;
        a2.Hq = p->heads_q;
        a2.qh = a.qh1;
        a2.oh = a.oh1;
        a2.lse_h = a.lse_h1;
        a2.U = p->batch * p->heads_q;
        a2.upx = a.grouped ? (int32_t)(G / X) * R : 0;
        a2.T = a.nsplit;
        plan->grid2 = (a.grouped ? X * a2.upx : a2.U) * a2.T;
    }
    return MFA_OK;
}

// Split-KV is chosen for decode-like calls: at most 256 query rows per
// sequence (one or two query tiles) and more keys than one chunk.  The chunk is a constant (2048 keys: on MI355X
// the best single size over B=1..64, Hq=16..32, Lk=8K..128K decode shapes).
// For varlen and B=1 calls the choice depends on the lengths only, so a
// sequence gets the same chunks alone (dense B=1) or inside a varlen batch
// and its rows are bit-identical either way.  A dense batch whose
// (sequence, head) units already fill the chip (>= 512 workgroups) runs the
// single pass: there the split's merge and extra workgroups cost ~8%.
constexpr int kSplitMaxLq = 256;
constexpr int kSplitKeys = 2048;
int auto_split_keys(const mfa_fwd_params* p, const ChipGeom& geom) {
    const int64_t kSplitMaxUnits = 2 * (int64_t)geom.cus;  // two workgroups per CU
    if (!p || p->dtype_in == MFA_DTYPE_F32 || p->tile_hint == MFA_TILE_PINGPONG ||
        p->tile_hint == MFA_TILE_PINGPONG256)
        return 0;
    if (p->seqlen_q > kSplitMaxLq || p->seqlen_k <= kSplitKeys) return 0;
    if (!p->cu_seqlens_q && p->batch > 1 && (int64_t)p->batch * p->heads_q >= kSplitMaxUnits) return 0;
    return kSplitKeys;
}

// Enqueue a planned split-KV call with its workspace `ws` (plan.ws_bytes
// bytes, 256-byte aligned): the chunk kernel writes every partial the merge
// kernel reads (each chunk of each row that exists, lse -inf and O 0 for a
// chunk without a valid key), so the workspace needs no clearing.
int launch_splitkv(Plan& plan, void* ws, hipStream_t st, const char* who) {
    KArgs& a = plan.args;
    // (the planned rows: a packed grouped-query decode has a.Lq = query heads
    // per K/V head rows per unit, not the caller's seqlen_q)
    const int64_t rows = (int64_t)a.nsplit * a.U * a.Lq;
    a.ws_o = static_cast<float*>(ws);
    a.ws_lse = a.ws_o + rows * a.ws_ld;
    plan.args2.ws_o = a.ws_o;
    plan.args2.ws_lse = a.ws_lse;
    // one chunk (every key range fits): the kernels store O themselves
    launch_plan(plan, st);
    if (a.nsplit > 1)
        hipLaunchKernelGGL(plan.combine, dim3((unsigned)((int64_t)a.U * a.Lq)), dim3(64), 0, st, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_err(MFA_ERR_LAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
    return MFA_OK;
}

}  // namespace

// Workspace of mfa_fwd_splitkv_static: one array per GPU (each device that
// loads the library's code object gets its own copy, held until the process
// ends).  In host code `scratch` only names the symbol; its device address on
// a device comes from hipGetSymbolAddress with that device current, looked up
// once per device and kept in g_scratch_ptr.
static __device__ __align__(256) unsigned char scratch[MFA_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 256;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];

// Device address of `scratch` on the device `st` belongs to (the current
// device for the null stream); the first call on a device looks it up with
// that device current.
int static_scratch(hipStream_t st, void** out) {
    int dev = -1;
    hipError_t e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return set_err(MFA_ERR_LAUNCH, "mfa_fwd_splitkv_static: no device for the stream: %s",
                                        hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxScratchDevices)
        return set_err(MFA_ERR_INVALID, "mfa_fwd_splitkv_static: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        void* ptr = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (cur >= 0 && cur != dev) {
            const hipError_t e2 = hipSetDevice(cur);
            if (e == hipSuccess) e = e2;
        }
        if (e != hipSuccess || !ptr)
            return set_err(MFA_ERR_LAUNCH, "mfa_fwd_splitkv_static: hipGetSymbolAddress(scratch) on device %d: %s",
                           dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return MFA_OK;
}

}  // namespace

char* mfa_error_buffer() { return g_err; }

extern "C" {

int mfa_abi_version(void) { return MFA_ABI_VERSION; }

int mfa_params_size(void) { return (int)sizeof(mfa_fwd_params); }

const char* mfa_last_error(void) { return g_err; }

int mfa_supported(int32_t dtype_in, int32_t head_dim) {
    if (dtype_in != MFA_DTYPE_F16 && dtype_in != MFA_DTYPE_BF16 && dtype_in != MFA_DTYPE_F32) return 0;
    return head_dim > 0 && head_dim <= MFA_MAX_HEAD_DIM && head_dim % 8 == 0;
}

int mfa_fwd_launch_info(const mfa_fwd_params* params, mfa_launch_info* info) {
    g_err[0] = 0;
    if (!info) return set_err(MFA_ERR_INVALID, "mfa_fwd_launch_info: info is NULL");
    Plan plan;
    const int rc = make_plan(params, &plan, chip_geometry_current());
    if (rc != MFA_OK) return rc;
    info->grid_x = plan.empty ? 0 : plan.grid;
    info->block_x = plan.cfg.threads;
    info->rows_per_block = plan.cfg.rows;
    info->keys_per_block = plan.cfg.keys;
    info->lds_bytes = plan.cfg.lds;
    snprintf(info->kernel_name, sizeof(info->kernel_name), "%s%s%s", plan.cfg.name,
             (params->softcap > 0.f || params->alibi_slopes) ? "+bias" : "", params->block_table ? "+paged" : "");
    return MFA_OK;
}

int32_t mfa_fwd_split_keys(const mfa_fwd_params* params) { return auto_split_keys(params, chip_geometry_current()); }

int64_t mfa_fwd_workspace_bytes(const mfa_fwd_params* params, int32_t split_keys) {
    g_err[0] = 0;
    if (split_keys == 0) return 0;
    Plan plan;
    const int rc = make_plan(params, &plan, chip_geometry_current(), split_keys);
    if (rc != MFA_OK) return rc;
    return plan.empty ? 0 : plan.ws_bytes;
}

int mfa_fwd_splitkv(const mfa_fwd_params* params, int32_t split_keys, void* workspace, int64_t workspace_bytes,
                    void* stream) {
    g_err[0] = 0;
    if (split_keys == 0) return mfa_fwd(params, stream);
    Plan plan;
    const int rc = make_plan(params, &plan, chip_geometry_of(static_cast<hipStream_t>(stream)), split_keys);
    if (rc != MFA_OK) return rc;
    if (plan.empty) return MFA_OK;
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
        return set_err(MFA_ERR_INVALID, "mfa_fwd_splitkv: workspace must be a 256-byte aligned device pointer");
    if (workspace_bytes < plan.ws_bytes)
        return set_err(MFA_ERR_INVALID, "mfa_fwd_splitkv: workspace of %lld bytes, %lld needed",
                       (long long)workspace_bytes, (long long)plan.ws_bytes);
    return launch_splitkv(plan, workspace, static_cast<hipStream_t>(stream), "mfa_fwd_splitkv");
}

int mfa_fwd_splitkv_static(const mfa_fwd_params* params, int32_t split_keys, void* stream) {
    g_err[0] = 0;
    if (split_keys == 0) return mfa_fwd(params, stream);
    Plan plan;
    const int rc = make_plan(params, &plan, chip_geometry_of(static_cast<hipStream_t>(stream)), split_keys);
    if (rc != MFA_OK) return rc;
    if (plan.empty) return MFA_OK;
    if (plan.ws_bytes > MFA_STATIC_SCRATCH_BYTES)
        return set_err(MFA_ERR_INVALID,
                       "mfa_fwd_splitkv_static: this call needs %lld bytes of workspace, more than the static "
                       "scratch's %lld; use mfa_fwd_splitkv with a caller workspace, or larger chunks",
                       (long long)plan.ws_bytes, (long long)MFA_STATIC_SCRATCH_BYTES);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = nullptr;
    const int src = static_scratch(st, &ws);
    if (src != MFA_OK) return src;
    return launch_splitkv(plan, ws, st, "mfa_fwd_splitkv_static");
}

int mfa_fwd(const mfa_fwd_params* params, void* stream) {
    g_err[0] = 0;
    Plan plan;
    const int rc = make_plan(params, &plan, chip_geometry_of(static_cast<hipStream_t>(stream)));
    if (rc != MFA_OK) return rc;
    if (plan.empty) return MFA_OK;
    launch_plan(plan, static_cast<hipStream_t>(stream));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_err(MFA_ERR_LAUNCH, "mfa_fwd: launch failed: %s", hipGetErrorString(e));
    return MFA_OK;
}

}  // extern "C"
