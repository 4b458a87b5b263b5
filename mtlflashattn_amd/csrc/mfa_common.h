// mfa_common.h -- definitions shared by the forward (mfa_fwd.hip) and
// backward (mfa_bwd.hip) kernels of libmtlfa_hip.so: operand types, the
// kernel argument block, the (sequence, head) views of the tensors, the
// paged-K/V block lookup and the valid key interval of a query
// (metal_flash_attn/_kernel.py:54-64).
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

// Thread-local message buffer behind mfa_last_error() (512 bytes, defined in
// mfa_fwd.hip), shared by every entry point of the library.
__attribute__((visibility("hidden"))) char* mfa_error_buffer();

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2_t;

constexpr float kLog2e = 1.4426950408889634f;
// dword 3 of a gfx9 buffer resource (raw buffer, 32-bit data format)
constexpr int kBufferDword3 = 0x00020000;

// Kernel argument block (copied by value into the kernarg segment).
struct KArgs {
    const char* q;
    const char* k;
    const char* v;
    char* o;
    // element strides
    int64_t qb, qs, qh;
    int64_t kb, ks, kh;
    int64_t vb, vs, vh;
    int64_t ob, os, oh;
    const int32_t* cu_q;
    const int32_t* cu_k;
    const float* alibi;
    int32_t alibi_bstride;
    int32_t B, Hq, Hkv, Lq, Lk, D;
    float scale;      // softmax scale
    float scale_log2; // scale * log2(e)
    float softcap;    // 0 = off
    float softcap_k;  // 2 * log2(e) / softcap
    float softcap_sk; // scale * softcap_k (the soft-cap of a raw score in one exponent)
    int32_t wl, wr, causal;
    int32_t decode_pack;  // rows are the query heads of one K/V head (single-row GQA decode)
    // varlen: element strides between the tokens of q / o at which sequences
    // start, and query rows per token (pack_r = query heads per K/V head when
    // packed, else 1; rows then step by qs / os)
    int64_t qts, ots;
    int32_t pack_r;
    // sequences of one query row (varlen calls that mix them with longer
    // ones): 0 = every sequence is this launch's, 1 = this launch skips them
    // (the exact-row kernel's launch computes them), 2 = this launch (the
    // exact-row kernel) computes only them
    int32_t single_rows;
    // ping-pong tiles packing the query heads of one K/V head (grouped-query
    // calls): hpack heads share a tile and its K/V stream, each taking
    // 1/hpack of the tile's rows at the same positions.  The unit heads Hq
    // are then groups of hpack heads (qh / oh / lse_h step a whole group) and
    // qh1 / oh1 / lse_h1 step one head inside it.  hpack = 1: one head.
    int32_t hpack;
    int64_t qh1, oh1, lse_h1;
    int32_t out_f32;
    // schedule
    int32_t T;        // query tiles per (sequence, head)
    int32_t U;        // (sequence, head) units = B * Hq
    int32_t upx;      // units per XCD (grouped schedule)
    int32_t grouped;  // 1: XCD-grouped by K/V head, 0: linear
    int32_t xcd_shift;  // log2 of the device's XCD count (grouped schedule)
    int32_t tile_major;  // grouped order within an XCD: 1 tile-major, 0 unit-major
    // split-KV: the key range of a sequence is cut into chunks of split_keys
    // keys (a multiple of the key block); workgroup (tile, split) writes the
    // chunk's normalised O and log2-sum-exp to the workspace, the combine
    // kernel merges them.  nsplit = chunks of the longest sequence (<= 1: off).
    int32_t nsplit;
    int32_t split_keys;
    int32_t ws_ld;    // floats per workspace O row (padded head dim)
    float* ws_o;      // [nsplit][U][Lq][ws_ld]
    float* ws_lse;    // [nsplit][U][Lq]
    // softmax log-sum-exp output (natural log; NULL = off), rows contiguous
    float* lse;
    int64_t lse_b, lse_h;
    // paged K/V: key j of sequence b is row j % page of page
    // bt[b * bt_b + j / page]; j / page = umulhi(j, page_m) >> page_s.
    // Contiguous K/V: bt = NULL, page_m = 0 (every key is in "page" 0, whose
    // id comes from a one-entry zero table).
    const int32_t* bt;
    int64_t bt_b;
    int32_t page, npages;
    uint32_t page_m;
    int32_t page_s;
};

// page table of contiguous K/V: one page with id 0
__device__ const int32_t kNoPages[1] = {0};

// ----------------------------------------------------------------------------
// small device helpers

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Store of a result the kernel never reads back (attention output O): a
// non-temporal (streaming) store, so the write does not hold L2 lines that
// the K/V stream reuses.  Measured on the O stores: config 4 -3.4 %,
// config 6 -4 %, configs 2-3 -0.4 %.
template <class T>
__device__ __forceinline__ void store_stream(T* p, const T& v) { __builtin_nontemporal_store(v, p); }

// Larger of a and b for scores that are never NaN (finite or -inf):
// IEEE maximum, which needs no NaN-quieting of its inputs (fmaxf's maxnum
// costs a canonicalising v_max_f32 per operand that is not a fresh
// arithmetic result, e.g. an MFMA accumulator or a cross-lane value).
__device__ __forceinline__ float fmax_nn(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// value of `x` in lane (lane ^ 32) and in this lane, combined by max
__device__ __forceinline__ float max_halves(float x) {
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return fmax_nn(__int_as_float(sw[0]), __int_as_float(sw[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return __int_as_float(sw[0]) + __int_as_float(sw[1]);
}

// Direct-to-LDS load (buffer_load_dwordx4 ... lds): lane i of the wave
// writes the 16 bytes at `off` of the resource to dst + 16*i bytes (dst is
// wave-uniform; an offset beyond the resource writes zeros).  Issued from
// inline asm: the compiler does not see an LDS write, so it adds no vmcnt(0)
// before later LDS reads it cannot prove disjoint.  The caller waits (vmcnt) before a
// barrier that publishes the data.  The resource is a raw buffer: base
// address, stride 0, `bytes` records, dword3 0x00020000.
// M0 carries the LDS address.  It is an input operand bound to M0 itself
// ("{m0}"): the compiler writes M0 before the statement and knows what it
// holds afterwards (the asm only reads it), so M0 is neither written by the
// asm nor in its clobber list.  (s_nop 0: one wait state between the M0
// write and the load that reads it.)
__device__ __forceinline__ void lds_load16(uint64_t base, uint32_t bytes, uint16_t* dst, uint32_t off) {
    typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t rsrc_t;
    const rsrc_t r = {(uint32_t)base, (uint32_t)(base >> 32) & 0xffffu, bytes, (uint32_t)kBufferDword3};
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)dst;
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(off), "s"(r), "{m0}"(lds)
                 : "memory");
}

// Compile-time loop: f(std::integral_constant<int, I>{}) for I = 0 .. N-1.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// ds_read_b64_tr_b16 at LDS byte address addr + OFF, issued from inline asm
// so the constant lands in the offset field.  The compiler does not track
// this load: the caller waits (lds_wait) before touching the result.
template <int OFF>
__device__ __forceinline__ u32x2_t lds_read_tr16(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "DS offset field");
    u32x2_t r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
    return r;
}
// Wait until at most N LDS operations are in flight; x and y (results of
// asynchronous LDS reads) are tied through the wait, so nothing reads or moves
// them before it.
template <int N, class T>
__device__ __forceinline__ void lds_wait(T& x, T& y) {
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(x), "+v"(y) : "n"(N));
}

// Empty asm that reads and rewrites x in registers: pure arithmetic can be
// moved across an asm barrier, but not across a pin of its inputs or outputs.
template <class T>
__device__ __forceinline__ void pin(T& x) {
    asm volatile("" : "+v"(x));
}

// Accumulator row of register r in the 32x32 MFMA C layout, minus the
// half-wave term 4*(lane/32): rows 8*(r/4) + r%4.
__device__ __forceinline__ constexpr int acc_row(int r) { return 8 * (r >> 2) + (r & 3); }

// Position of key kk (0..31 inside a 32-key group) in the V^T LDS rows:
// bits 2 and 3 swapped, so that the 8 keys one half-wave feeds to one
// PV MFMA (accumulator registers 8*st..8*st+7) are contiguous.
__device__ __forceinline__ int vt_pos(int kk) {
    return (kk & ~12) | ((kk & 4) << 1) | ((kk & 8) >> 1);
}

// Map the linear workgroup id to (sequence, q head, query tile).
// Returns false for padding workgroups.
__device__ __forceinline__ bool decode_tile(const KArgs& a, int bid, int& b, int& hq, int& t) {
    int unit, tt;
    if (a.grouped) {
        // workgroup ids are dealt round-robin over the X = 2^xcd_shift XCDs
        // (8 on MI355X); XCD x owns the
        // K/V head groups g = b*Hkv + hkv with g % X == x, all their q heads
        // and all their tiles.  Within an XCD the order is unit-major (all
        // tiles of one (sequence, q head), heaviest first, then the next), so
        // the workgroups resident on the XCD share one head's K/V in its L2,
        // or, with a.tile_major (the plan sets it for causal and windowed
        // calls, except head-packed varlen ones), tile-major: the heaviest
        // tiles of every unit first, so the XCD's CUs take the work longest
        // first and finish together.
        const int xcd = bid & ((1 << a.xcd_shift) - 1);
        const int slot = bid >> a.xcd_shift;
        int j;
        if (a.tile_major) {
            tt = slot / a.upx;
            j = slot - tt * a.upx;
        } else {
            j = slot / a.T;
            tt = slot - j * a.T;
        }
        const int R = a.Hq / a.Hkv;
        const int jg = j / R;
        const int g = xcd + (jg << a.xcd_shift);
        const int r = j - jg * R;
        b = g / a.Hkv;
        const int hkv = g - b * a.Hkv;
        hq = hkv * R + r;
        unit = b * a.Hq + hq;
        if (unit >= a.U) return false;
    } else {
        tt = bid / a.U;
        unit = bid - tt * a.U;
        b = unit / a.Hq;
        hq = unit - b * a.Hq;
    }
    t = a.T - 1 - tt;  // heaviest (last) query tiles first
    return t >= 0;
}

struct SeqView {
    const char* q;
    const char* k;  // K/V of this head: sequence start, or page 0 when paged
    const char* v;
    char* o;
    float* lse;            // this (sequence, head)'s softmax_lse row, or NULL
    const int32_t* bt;     // this sequence's page table row (kNoPages: contiguous)
    int Lq, Lk;
};

// ES: input element bytes; the output element size follows a.out_f32.
template <int ES>
__device__ __forceinline__ SeqView seq_view(const KArgs& a, int b, int hq) {
    SeqView s;
    const int OES = a.out_f32 ? 4 : ES;
    const int hkv = hq / (a.Hq / a.Hkv);  // grouped-query mapping (_kernel.py:54)
    int64_t qo, ko;
    if (a.cu_q) {
        const int q_start = a.cu_q[b];
        const int k_start = a.cu_k[b];
        s.Lq = (a.cu_q[b + 1] - q_start) * a.pack_r;
        s.Lk = a.cu_k[b + 1] - k_start;
        qo = (int64_t)q_start * a.qts;
        ko = a.bt ? 0 : (int64_t)k_start;  // paged: pages come from the table
        s.q = a.q + (qo + (int64_t)hq * a.qh) * ES;
        s.k = a.k + (ko * a.ks + (int64_t)hkv * a.kh) * ES;
        s.v = a.v + (ko * a.vs + (int64_t)hkv * a.vh) * ES;
        s.o = a.o + ((int64_t)q_start * a.ots + (int64_t)hq * a.oh) * OES;
        s.lse = a.lse ? a.lse + (int64_t)hq * a.lse_h + q_start : nullptr;
    } else {
        s.Lq = a.Lq;
        s.Lk = a.Lk;
        const int64_t kb = a.bt ? 0 : (int64_t)b;  // paged: batch stride = page stride
        s.q = a.q + ((int64_t)b * a.qb + (int64_t)hq * a.qh) * ES;
        s.k = a.k + (kb * a.kb + (int64_t)hkv * a.kh) * ES;
        s.v = a.v + (kb * a.vb + (int64_t)hkv * a.vh) * ES;
        s.o = a.o + ((int64_t)b * a.ob + (int64_t)hq * a.oh) * OES;
        s.lse = a.lse ? a.lse + (int64_t)b * a.lse_b + (int64_t)hq * a.lse_h : nullptr;
    }
    s.bt = a.bt ? a.bt + (int64_t)b * a.bt_b : kNoPages;
    return s;
}

// Element offset from sv.k (bstride = a.kb, sstride = a.ks) or sv.v of the
// first row of the key block starting at key j, and whether that block may be
// read.  Paged K/V: row j % page of page bt[j / page]; a block never straddles
// pages (pages hold a multiple of 256 keys, blocks start at multiples of their
// size, which divides 256).  The table index is clamped to the last key below
// kend, so the prefetch of a block past the sequence reads no entry beyond the
// sequence's own; a page id outside [0, npages) makes the block unreadable.
// Contiguous K/V (PAGED false, a separate kernel instantiation): j * sstride,
// with no table read -- the scalar load's wait (lgkmcnt) would also wait for
// every LDS read in flight.  All values are wave-uniform, without branches.
template <bool PAGED>
__device__ __forceinline__ int64_t kv_block_off(const KArgs& a, const SeqView& sv, int j, int kend, int64_t bstride,
                                                int64_t sstride, bool& ok) {
    if constexpr (!PAGED) {
        ok = true;
        return (int64_t)j * sstride;
    }
    const uint32_t jj = (uint32_t)min(j, max(kend - 1, 0));
    const int idx = (int)(__umulhi(jj, a.page_m) >> a.page_s);
    // read-only during the kernel: a constant-address-space load (scalar unit)
    const int pg = ((const __attribute__((address_space(4))) int32_t*)(uintptr_t)sv.bt)[idx];
    ok = (uint32_t)pg < (uint32_t)a.npages;
    return (int64_t)(ok ? pg : 0) * bstride + (int64_t)(j - idx * a.page) * sstride;
}

// tanh to within 2 ulp: the odd Taylor series of tanh through t^17 below
// |y| = 0.6 (the next term is below 3e-8 of the result there), and
// 1 - 2 / (exp(2|y|) + 1) above it, where the difference no longer cancels
// (the exponential form loses the small values' relative precision: near
// y = 0 it is off by up to 1.4e-7 absolute)
__device__ __forceinline__ float precise_tanh(float y) {
    const float t = fabsf(y);
    float r;
    if (t < 0.6f) {
        const float u = t * t;
        float p = 6404582.f / 10854718875.f;  // coefficients of t^17, t^15, ..., t^3
        p = fmaf(p, u, -929569.f / 638512875.f);
        p = fmaf(p, u, 21844.f / 6081075.f);
        p = fmaf(p, u, -1382.f / 155925.f);
        p = fmaf(p, u, 62.f / 2835.f);
        p = fmaf(p, u, -17.f / 315.f);
        p = fmaf(p, u, 2.f / 15.f);
        p = fmaf(p, u, -1.f / 3.f);
        r = fmaf(t * u, p, t);
    } else {
        r = 1.f - __fdiv_rn(2.f, fast_exp2(t * (2.f * kLog2e)) + 1.f);
    }
    return copysignf(r, y);
}


// Valid key interval [lo, hi] of the query with bottom-right center `c`
// (_kernel.py:56-64).  Window bounds are clamped on the host so c+wr cannot
// overflow.
__device__ __forceinline__ int key_lo(const KArgs& a, int c) { return a.wl >= 0 ? max(c - a.wl, 0) : 0; }
__device__ __forceinline__ int key_hi(const KArgs& a, int c, int Lk) {
    int hi = Lk - 1;
    if (a.causal) hi = min(hi, c);
    if (a.wr >= 0) hi = min(hi, c + a.wr);
    return hi;
}


}  // namespace
