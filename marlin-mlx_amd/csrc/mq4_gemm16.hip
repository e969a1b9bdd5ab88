// Prefill-shaped (large M) MLX-affine Q4 GEMM for gfx950 with the weights
// dequantized to fp16 in registers and fed to the fp16 MFMA.
//
// Same call sites as mq4_gemm.hip: qmatmul (src/model/marlin.cpp:18-25)
// inside mlp_forward (:31-35) over all S prompt tokens, with the rms_norm in
// front (:141, :12-16) and the swiglu (:27-29) fused in; used for both
// products of mq4_mlp_residual: gate/up with the SwiGLU epilogue, and down
// with the residual add (:142), whole or in K parts whose fp32 sums
// kpart_residual_kernel adds in order.
//
//   Y[M, N] = X[M, K] . W[N, K]^T,  W[n, k] = s[n, g] * q[n, k] + b[n, g],  g = k / 64
//
// mq4_gemm.hip keeps both MFMA operands exact (x and 128 + q in bf16) and
// folds every group into the fp32 result with the VALU, two instructions per
// output and group: at 64 x 64 outputs per wave that fold is as long as the
// group's MFMAs, and the kernel is VALU-bound.  Here each weight is formed
// once as w = fp16(s q + b), one rounding (v_pk_fma_f16 on exact fp16 q, s
// and b), and the MFMA accumulates x . w straight into the result: no fold.
// s q + b of a bf16 scale and bias and a 4-bit q mostly fits fp16's 11-bit
// significand, so most weights are exact; on 0.02-std Gaussian weights the
// product's error is 2.4e-6 of the output rms (max 1.5e-4), against about
// 1e-5 for the exact-operand kernel's fp32 fold.  Scales and biases convert
// to fp16 exactly in its normal range (beyond 65504 a weight would not be
// finite; below 2^-14 the conversion is subnormal, an absolute error under
// 2^-25).
//
// The activations are an fp16 copy of the bf16 operand in the MFMA pair
// order (launch_pair_rows16: normalized x), each row scaled by a power of two
// 2^-e (e = 0 unless the row holds values of 2^15 or more) that the epilogue
// multiplies back exactly, so any bf16 input stays finite.  A bf16 value
// converts to fp16 exactly unless it lies below 2^-14 (2^-14 + e), where
// fp16 is subnormal: an absolute error under 2^-25 of the row's scale.
//
// Work decomposition:
//  * A 256-thread block computes 128 rows x 256 weight columns (one matrix:
//    256 output columns; gate and up: 128 output columns each, for the fused
//    SwiGLU); wave w takes all 128 rows and 64 weight columns (gate/up:
//    32 gate and the same 32 up columns) as 4 x 2 v_mfma_f32_32x32x16_f16
//    tiles, so each weight is dequantized once per block, by the one wave
//    that uses it (about two VALU per weight: a v_and_or_b32 forms two fp16
//    1024 + q, a v_pk_add_f16 takes the 1024 off, a v_pk_fma_f16 applies s
//    and b to the pair).
//  * Per 64-k group, the 128 x 64 activations (16 KB, each row's eight
//    16-byte chunks XOR-swizzled by (row / 2) % 8: the 16 lanes of a
//    ds_read_b128 phase, 16 rows at one chunk, cover the 64 banks once) and
//    the 256 x 32 bytes of packed weights (per 32 columns one DMA
//    instruction, lane l reading k-half l / 32 of column l % 32, so that the
//    stage holds each k-half's 32 columns in consecutive slots) go to LDS by
//    DMA, two stages, one group ahead;
//    the columns' scales and biases follow every eight groups (16 bytes per
//    column, two slots).  Each step waits for all of its wave's DMA;
//    barriers carry no memory fence.  (Per-group DMA of the scales, four
//    bytes from 64 columns per instruction, and of one k-half of 64 columns
//    made the kernel bound by L2 requests: 17.5 M per gate/up call at M =
//    2048.)
//  * The operand layout is mq4_gemm.hip's: lane l of a tile holds row (or
//    weight column) l % 32 and k-half l / 32; MFMA step ks takes word ks of
//    the half, whose nibble pairs (q_p, q_{p+4}) meet the activations in the
//    pair order (x_p, x_{p+4}) of the pre-pass.  The weights are the MFMA's
//    row operand and the activations its column operand, so that a result
//    lane holds one activation row and four runs of four consecutive weight
//    columns: the epilogue reads one row scale per 32 rows and writes 8-byte
//    runs.  (With the activations as the row operand a lane held one column
//    of 16 rows: a row-scale load and a 2-byte store per output, which cost
//    the SwiGLU product 26 us of 72 at M = 2048 in a copy without the
//    dequantization and the data movement.)
#include <type_traits>

#include "mq4_device.h"
#include "mq4_gemm.h"
#include "mq4_host.h"

namespace mq4 {

namespace g16 {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kNW = 4;                    // waves per block
constexpr int kThreads = 64 * kNW;
constexpr int TBM = 128;                  // rows per block
constexpr int A_I = TBM * 8 / (64 * kNW); // activation DMA instructions per wave and group (4)

// NJ 32-column MFMA tiles per wave: a block covers BNW = 32 NJ kNW weight
// columns (NJ = 2: 256, two blocks per CU; NJ = 1: 128, three blocks per CU).
template <int NJ>
struct Cols {
    static constexpr int BNW = 32 * NJ * kNW;          // weight columns per block
    static constexpr int B_I = 2 * BNW / 64 / kNW;     // weight DMA instructions per wave and group (NJ)
    static constexpr int SB_I = 2 * BNW / (64 * kNW);  // scale/bias DMA instructions per wave and 8 groups (NJ)
};

template <int NJ>
struct Stage {
    uint4 a[TBM * 8];                     // [row][chunk ^ ((row >> 1) & 7)], fp16 pairs
    uint4 b[2 * Cols<NJ>::BNW];           // [32-column block][k-half][column]
};
// Scales and biases of 8 groups: [scales | biases][weight column], 16 bytes
// (groups 8 t .. 8 t + 7) each.
template <int NJ>
struct SbStage {
    uint4 v[2][Cols<NJ>::BNW];
};
static_assert(2 * sizeof(Stage<2>) + 2 * sizeof(SbStage<2>) <= 65536, "LDS DMA targets must lie in the first 64 KiB");
static_assert(3 * (2 * sizeof(Stage<1>) + 2 * sizeof(SbStage<1>)) <= 160 * 1024, "three NJ = 1 blocks per CU");

__device__ __forceinline__ void lds_dma16(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}
__device__ __forceinline__ void lds_dma4(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds(src, lds, 4, 0, 0);
}

// bf16 bits -> fp16 (round to nearest even; exact for bf16 values of fp16's
// normal range)
__device__ __forceinline__ _Float16 bf16_to_h(uint32_t bits) { return (_Float16)bf16_to_f32(bits); }

// (s & m) | c in one v_and_or_b32, the mask in an SGPR and the exponent
// bits in a VGPR, both set up once by the caller: the nibbles m selects in
// each 16-bit half as fp16 mantissa bits under c's exponents.
__device__ __forceinline__ uint32_t nib_pair_h(uint32_t s, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(s), "s"(m), "v"(c));
    return r;
}

// The eight fp16 weights fp16(s q + b) of one packed word, in the nibble-pair
// order (q0, q4), (q1, q5), (q2, q6), (q3, q7).  Pairs 0 and 2 are the low
// nibbles of each half of w and of w >> 8, under the exponent of 1024 (fp16
// 1024 + q); pairs 1 and 3 are their high nibbles, left in place (bits 4-7
// of the half) under the exponent of 64, whose mantissa step is 1/16 (fp16
// 64 + q): one shift per word instead of three.  m_lo / c_lo = 0x000f000f /
// 0x64006400, m_hi / c_hi = 0x00f000f0 / 0x54005400.
__device__ __forceinline__ h8_t dequant_word(uint32_t w, h2_t s2, h2_t b2, uint32_t m_lo, uint32_t c_lo,
                                             uint32_t m_hi, uint32_t c_hi) {
    const h2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const h2_t k64 = {(_Float16)64.0f, (_Float16)64.0f};
    const uint32_t w8 = w >> 8;
    const h2_t q[4] = {__builtin_bit_cast(h2_t, nib_pair_h(w, m_lo, c_lo)) - k1024,      // exact
                       __builtin_bit_cast(h2_t, nib_pair_h(w, m_hi, c_hi)) - k64,
                       __builtin_bit_cast(h2_t, nib_pair_h(w8, m_lo, c_lo)) - k1024,
                       __builtin_bit_cast(h2_t, nib_pair_h(w8, m_hi, c_hi)) - k64};
    uint32_t out[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) out[p] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q[p], s2, b2));
    return __builtin_bit_cast(h8_t, make_uint4(out[0], out[1], out[2], out[3]));
}

// Column of an 8-column chunk whose pair-order position (2 (c % 4) + c / 4)
// is r.
__device__ __forceinline__ int perm8(int r) { return 4 * (r & 1) + (r >> 1); }

// MFMA results are read by the VALU only in the epilogue; the padding keeps
// the wait states between the last MFMA and that read generous.
__device__ __forceinline__ void mfma_result_pad() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    __builtin_amdgcn_sched_barrier(0);
}

template <int EPI, int NJ>
__global__ __launch_bounds__(kThreads, NJ == 1 ? 3 : 2) void q4_gemm16_kernel(Gemm16Args p) {
#pragma clang fp contract(off)
    static_assert(EPI == GEMM_SWIGLU || EPI == GEMM_RESIDUAL, "the epilogues of mq4_mlp_residual");
    static_assert(NJ == 2 || (NJ == 1 && EPI == GEMM_RESIDUAL), "SwiGLU: a gate and an up tile per wave");
    constexpr int NMAT = EPI == GEMM_SWIGLU ? 2 : 1;
    constexpr int BNW = Cols<NJ>::BNW, B_I = Cols<NJ>::B_I, SB_I = Cols<NJ>::SB_I;
    constexpr int BN = BNW / NMAT;                       // output columns per block
    using Stage = g16::Stage<NJ>;
    using SbStage = g16::SbStage<NJ>;
    // one LDS object, stages first: the DMA targets stay in the first 64 KiB
    // (SwiGLU: the 8 KB SiLU table after them, read only by the epilogue)
    struct Smem {
        Stage st[2];
        SbStage sb[2];
        uint16_t lut[EPI == GEMM_SWIGLU ? SILU_LUT_N : 2];
    };
    __shared__ Smem smem;
    Stage &st0 = smem.st[0], &st1 = smem.st[1];
    SbStage &sb0 = smem.sb[0], &sb1 = smem.sb[1];
    static_assert(2 * sizeof(Stage) + 2 * sizeof(SbStage) <= 65536, "LDS DMA targets in the first 64 KiB");

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, col = lane & 31;
    const int M = p.M, N = p.N, K = p.K, G = K / 64;
    // K parts (GEMM_RESIDUAL): block b takes part b / tiles, groups
    // [part GL, (part + 1) GL), and writes its fp32 partial product
    const int S = EPI == GEMM_RESIDUAL && p.ksplit > 1 ? p.ksplit : 1;
    const int GL = G / S;
    int bt = blockIdx.x, kpart = 0;
    if (S > 1) {
        const int tiles = (int)gridDim.x / S;
        kpart = bt / tiles;
        bt -= kpart * tiles;
    }

    // XCD-aware block order: with the column blocks a multiple of 8, XCD x
    // (block b runs on XCD b % 8) takes a fixed eighth of them for every row
    // block, so its weights stay in its own L2
    const int NB = (N + BN - 1) / BN;
    int nb, mb;
    {
        const int b = bt;
        if ((NB & 7) == 0) {
            const int per = NB >> 3, s = b >> 3;
            nb = (s % per) * 8 + (b & 7);
            mb = s / per;
        } else {
            nb = b % NB;
            mb = b / NB;
        }
    }
    const int n0 = nb * BN, m0 = mb * TBM;

    // ---- DMA sources: wave-uniform bases plus 32-bit lane byte offsets ----
    const char* const xbase = reinterpret_cast<const char*>(p.x) + (int64_t)kpart * GL * 128;
    uint32_t aoff[A_I];
#pragma unroll
    for (int t = 0; t < A_I; ++t) {
        const int slot = (wave * A_I + t) * 64 + lane;
        const int r = slot >> 3, c = (slot & 7) ^ ((r >> 1) & 7);
        const int row = (m0 + r) < M ? (m0 + r) : (M - 1);
        aoff[t] = (uint32_t)(((int64_t)row * K + c * 8) * 2);
    }
    // weight column r of the block -> matrix and output row (rows past N
    // repeat row N - 1, never stored)
    auto wrow_of = [&](int r) -> int {
        const int n = NMAT == 2 ? n0 + (r % (BNW / 2)) : n0 + r;
        return n < N ? n : N - 1;
    };
    auto mat_of = [&](int r) -> const QMat& { return (NMAT == 2 && r >= BNW / 2) ? p.B : p.A; };
    // packed weights: instruction t covers 32 weight columns, lane l takes
    // k-half l / 32 of column l % 32 (its group's 32 bytes as two 16-byte
    // halves), so the stage holds [32-column block][k-half][column] and the
    // operand reads of a k-half are 32 consecutive 16-byte slots
    const char* bbase[B_I];
    uint32_t boff[B_I];
#pragma unroll
    for (int t = 0; t < B_I; ++t) {
        const int r0 = (wave * B_I + t) * 32;
        bbase[t] = reinterpret_cast<const char*>(mat_of(r0).wq) + (int64_t)kpart * GL * 32;
        boff[t] = (uint32_t)((int64_t)wrow_of(r0 + (lane & 31)) * (K / 2) + (lane >> 5) * 16);
    }
    // scales and biases: 16 bytes (8 groups) of one weight column per lane
    const char* sbbase[SB_I];
    uint32_t sboff[SB_I];
#pragma unroll
    for (int t = 0; t < SB_I; ++t) {
        const int u0 = (wave * SB_I + t) * 64, sel = u0 / BNW, r0 = u0 % BNW;
        sbbase[t] = reinterpret_cast<const char*>(sel ? mat_of(r0).b : mat_of(r0).s) + (int64_t)kpart * (GL / 8) * 16;
        sboff[t] = (uint32_t)((int64_t)wrow_of(r0 + lane) * G * 2);
    }
    auto issue = [&](int g, Stage& st) {
#pragma unroll
        for (int t = 0; t < A_I; ++t) lds_dma16(xbase + g * 128 + aoff[t], &st.a[(wave * A_I + t) * 64]);
#pragma unroll
        for (int t = 0; t < B_I; ++t) lds_dma16(bbase[t] + g * 32 + boff[t], &st.b[(wave * B_I + t) * 64]);
    };
    auto issue_sb = [&](int t8, SbStage& sbs) {        // groups 8 t8 .. 8 t8 + 7
#pragma unroll
        for (int t = 0; t < SB_I; ++t) lds_dma16(sbbase[t] + t8 * 16 + sboff[t], &sbs.v[0][(wave * SB_I + t) * 64]);
    };

    // ---- this lane's weight columns (block-relative) of tiles j = 0, 1 ----
    // Weight column c of a tile is MFMA row c, except for outputs in the
    // pair order: there MFMA row 8 b + r holds column 8 b + perm8(r), so that
    // the four consecutive MFMA rows of a result lane are four consecutive
    // positions of the pair order.
    const bool f16_out = EPI == GEMM_SWIGLU && p.yscale != 0.0f;
    const bool paired_out = EPI == GEMM_SWIGLU && !f16_out && p.ysum != nullptr;
    const int ccol = f16_out || paired_out ? ((col & ~7) | perm8(col & 7)) : col;
    int wr[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) wr[j] = NMAT == 2 ? j * (BNW / 2) + wave * 32 + ccol : wave * (32 * NJ) + j * 32 + ccol;

    uint32_t nib_mask, nib_exp, nib_mask_hi, nib_exp_hi;   // the nibble-pair constants, set up once
    asm("s_mov_b32 %0, 0x000f000f" : "=s"(nib_mask));
    asm("v_mov_b32 %0, 0x64006400" : "=v"(nib_exp));
    asm("s_mov_b32 %0, 0x00f000f0" : "=s"(nib_mask_hi));
    asm("v_mov_b32 %0, 0x54005400" : "=v"(nib_exp_hi));

    f32x16_t acc[4][NJ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // this group's packed words, scales and biases (read before the step's
    // DMA is issued, so no wait for it can come between)
    struct Wts {
        uint4 bw[NJ];
        h2_t s2[NJ], b2[NJ];
    };
    auto load_wts = [&](int g, const Stage& st) -> Wts {
        Wts w;
        const SbStage& sbs = ((g >> 3) & 1) ? sb1 : sb0;
        const int sh16 = (g & 1) * 16, dw = (g >> 1) & 3;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            w.bw[j] = st.b[(wr[j] >> 5) * 64 + h * 32 + (wr[j] & 31)];
            const _Float16 s = bf16_to_h((reinterpret_cast<const uint32_t*>(&sbs.v[0][wr[j]])[dw] >> sh16) & 0xffffu);
            const _Float16 b = bf16_to_h((reinterpret_cast<const uint32_t*>(&sbs.v[1][wr[j]])[dw] >> sh16) & 0xffffu);
            w.s2[j] = (h2_t){s, s};
            w.b2[j] = (h2_t){b, b};
        }
        return w;
    };
    // The weights are the MFMA row operand and the activations the column
    // operand: result lane l of tile (i, j) holds activation row i 32 + l % 32.
    // MFMA step ks + 1's activation reads and dequantization are issued
    // during step ks's MFMAs (two operand sets), one MFMA per LDS read and
    // four VALU.
    auto compute = [&](const Wts& wt, const Stage& st) {
        const uint4* bw = wt.bw;
        const h2_t* s2 = wt.s2;
        const h2_t* b2 = wt.b2;
        auto read_a = [&](int ks, h8_t (&a)[4]) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = i * 32 + col, ch = 4 * h + ks;
                a[i] = __builtin_bit_cast(h8_t, st.a[r * 8 + (ch ^ ((r >> 1) & 7))]);
            }
        };
        auto dequant = [&](int ks, h8_t (&bo)[NJ]) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const uint32_t w = ks == 0 ? bw[j].x : ks == 1 ? bw[j].y : ks == 2 ? bw[j].z : bw[j].w;
                bo[j] = dequant_word(w, s2[j], b2[j], nib_mask, nib_exp, nib_mask_hi, nib_exp_hi);
            }
        };
        auto mfmas = [&](const h8_t (&a)[4], const h8_t (&bo)[NJ]) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bo[j], a[i], acc[i][j], 0, 0, 0);
        };
        auto interleave = [] {
#pragma unroll
            for (int m = 0; m < 4 * NJ; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // MFMA
                if (m < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);      // LDS read
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);                 // VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        h8_t a0[4], a1[4], w0[NJ], w1[NJ];
        read_a(0, a0);
        dequant(0, w0);
        read_a(1, a1);
        dequant(1, w1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(a0, w0);
        read_a(2, a0);
        dequant(2, w0);
        interleave();
        mfmas(a1, w1);
        read_a(3, a1);
        dequant(3, w1);
        interleave();
        mfmas(a0, w0);
        mfmas(a1, w1);
    };
    // Two stages: step g waits for all of this wave's DMA (group g's), meets
    // the other waves at the barrier, reads group g's weights, issues group
    // g + 1 into the stage read in step g - 1 (past the end: the last group
    // again, into a stage nobody reads), at every eighth group also the next
    // eight groups' scales and biases into the slot read by the eight groups
    // before, and computes group g.
    auto step = [&](int g, const Stage& cur, Stage& nxt) {
        wait_vmcnt<0>();
        lds_barrier();                               // group g is in `cur` for every wave
        const Wts wt = load_wts(g, cur);
        issue(g + 1 < GL ? g + 1 : g, nxt);          // into the stage read in step g - 1
        if ((g & 7) == 0 && g + 8 < GL) issue_sb((g >> 3) + 1, ((g >> 3) & 1) ? sb0 : sb1);
        compute(wt, cur);
    };
    // the SiLU table (SwiGLU) is loaded with group 0 and stored to LDS after
    // its wait; the first step's barrier publishes it
    uint4 lut0 = make_uint4(0, 0, 0, 0), lut1 = lut0;
    if (EPI == GEMM_SWIGLU) {
        static_assert(SILU_LUT_N * 2 == 2 * 16 * kThreads, "two 16-byte pieces of the table per thread");
        const uint4* src = reinterpret_cast<const uint4*>(p.silu_lut);
        lut0 = src[tid];
        lut1 = src[tid + kThreads];
    }
    issue(0, st0);
    issue_sb(0, sb0);
    if (EPI == GEMM_SWIGLU) {
        wait_vmcnt<0>();
        uint4* dst = reinterpret_cast<uint4*>(smem.lut);
        dst[tid] = lut0;
        dst[tid + kThreads] = lut1;
    }
    int g0 = 0;
    for (; g0 + 2 <= GL; g0 += 2) {
        step(g0, st0, st1);
        step(g0 + 1, st1, st0);
    }
    if (g0 < GL) step(g0, st0, st1);
    wait_vmcnt<0>();                                 // no DMA outstanding past the loop
    mfma_result_pad();

    // ---- epilogue: result lane l of tile (i, j) holds activation row
    // i 32 + l % 32 and MFMA rows (e / 4) 8 + (l / 32) 4 + e % 4 of tile j:
    // four runs of four consecutive output columns (natural order, or the
    // pair-order positions 4 (l / 32) .. + 3 of an 8-column chunk), each
    // stored as one 8-byte (16 for fp32) write.
    // SwiGLU with ysum: h also goes to an LDS tile in natural column order,
    // 64 rows at a time (stage 0, free once every wave is past its last
    // group), for the group sums of its rows.
    constexpr int TS = BN + 8;                                     // bf16 per epilogue tile row
    uint16_t* tile = reinterpret_cast<uint16_t*>(&st0);          // [64][TS] bf16
    static_assert(64 * (BNW / 2 + 8) * 2 <= (int)sizeof(Stage), "epilogue tile");
    // whole-run vector stores: N % 4 == 0 and 8-byte aligned y and res
    // (16-byte aligned fp32 parts)
    const bool vec = N % 4 == 0 &&
                     (S > 1 ? reinterpret_cast<uintptr_t>(p.part) % 16 == 0
                            : reinterpret_cast<uintptr_t>(p.y) % 8 == 0 &&
                                  (EPI != GEMM_RESIDUAL || reinterpret_cast<uintptr_t>(p.res) % 8 == 0));
    const float ascale = p.ascale != 0.0f ? p.ascale : 1.0f;
    // The lane's four row scales, loaded together (one wait, not one per
    // row tile).
    float scv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + i * 32 + col;
        scv[i] = (p.xscale && row < M ? p.xscale[row] : 1.0f) * ascale;
    }
    // One-part residual epilogue: the residual runs of all four row tiles
    // are loaded before the first is written (one wait, not one per run).
    // In place (res == y) every element is read and written by the same
    // lane, the read first.
    const bool res_runs = EPI == GEMM_RESIDUAL && S == 1;
    uint2 resv[4][4 * NJ];
    const bool res_whole = vec && n0 + BN <= N;          // every run of the block: one 8-byte load
    auto load_res = [&](int i, uint2 (&rv)[4 * NJ]) {
        const int row = m0 + i * 32 + col;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int eg = 0; eg < 4; ++eg) {
                const int cb = n0 + wave * (32 * NJ) + j * 32 + eg * 8 + h * 4;
                uint2 t = make_uint2(0u, 0u);
                if (row < M && cb < N) {
                    const uint16_t* r = p.res + (int64_t)row * N + cb;
                    if (vec && cb + 3 < N) {
                        t = *reinterpret_cast<const uint2*>(r);
                    } else {
                        uint32_t e[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) e[q] = cb + q < N ? r[q] : 0u;
                        t = make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
                    }
                }
                rv[j * 4 + eg] = t;
            }
    };
    if (res_runs) {
        if (res_whole) {
            // rows past M read row M - 1 (never stored): no branch between
            // the loads
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = m0 + i * 32 + col;
                const uint16_t* r = p.res + (int64_t)(row < M ? row : M - 1) * N + n0 + wave * (32 * NJ) + h * 4;
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int eg = 0; eg < 4; ++eg)
                        resv[i][j * 4 + eg] = *reinterpret_cast<const uint2*>(r + j * 32 + eg * 8);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) load_res(i, resv[i]);
        }
    }
    // One wait for the row scales and residual runs, before the first branch
    // of the epilogue: past it the compiler's waits at branch joins would
    // count this tile's stores and drain them.
    wait_vmcnt<0>();
    auto emit = [&](int i, int rbase) {
        const int rl = i * 32 + col, row = m0 + rl;
        if (row >= M) return;
        const float sc = scv[i];
        const int64_t rowo = (int64_t)row * N;
        // SwiGLU of the lane's 16 (gate, up) pairs of this tile row
        uint32_t hv[16];
        if (EPI == GEMM_SWIGLU) {
            float ga[16], ua[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                ga[e] = acc[i][0][e] * sc;
                ua[e] = acc[i][1][e] * sc;
            }
            swiglu_bf16_lut_batch<16>(ga, ua, hv, smem.lut);
        }
#pragma unroll
        for (int j = 0; j < (NMAT == 2 ? 1 : NJ); ++j) {
#pragma unroll
            for (int eg = 0; eg < 4; ++eg) {
                const int cl = (NMAT == 2 ? wave * 32 : wave * (32 * NJ) + j * 32) + eg * 8 + h * 4;
                const int cb = n0 + cl;                             // first column (position) of the run
                if (cb >= N) continue;
                const bool whole = vec && cb + 3 < N;
                if (EPI == GEMM_SWIGLU) {
                    uint32_t o[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t v = hv[eg * 4 + q];
                        o[q] = v;
                        if (paired_out) tile[(rl - rbase) * TS + (cl & ~7) + perm8(h * 4 + q)] = (uint16_t)v;
                        if (f16_out) {
                            // exact for |h| within [2^-14, 65504] / yscale
                            const float hv = fminf(fmaxf(bf16_to_f32(v) * p.yscale, -65504.0f), 65504.0f);
                            o[q] = __builtin_bit_cast(uint16_t, (_Float16)hv);
                        }
                    }
                    uint16_t* y = reinterpret_cast<uint16_t*>(p.y) + rowo + cb;
                    if (whole) {
                        *reinterpret_cast<uint2*>(y) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            if (cb + q < N) y[q] = (uint16_t)o[q];
                    }
                    continue;
                }
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = acc[i][j][eg * 4 + q] * sc;
                if (S > 1) {
                    float* y = p.part + (int64_t)kpart * M * N + rowo + cb;
                    if (whole) {
                        *reinterpret_cast<float4*>(y) = make_float4(v[0], v[1], v[2], v[3]);
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            if (cb + q < N) y[q] = v[q];
                    }
                    continue;
                }
                uint32_t o[4];
                uint16_t* y = reinterpret_cast<uint16_t*>(p.y) + rowo + cb;
                const uint2 t = resv[i][j * 4 + eg];
                const uint32_t rv[4] = {t.x & 0xffffu, t.x >> 16, t.y & 0xffffu, t.y >> 16};
#pragma unroll
                for (int q = 0; q < 4; ++q) o[q] = f32_to_bf16(bf16_to_f32(rv[q]) + round_bf16(v[q]));
                if (whole) {
                    *reinterpret_cast<uint2*>(y) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (cb + q < N) y[q] = (uint16_t)o[q];
                }
            }
        }
    };
    // ysum of group n0 / 64 + gi of rows rbase .. rbase + 63: thread t takes
    // row t / 4, group (t / 2) % 2 and half t % 2 (32 values summed left to
    // right), then the two halves are added (the order of mq4_gemm.hip's
    // paired SwiGLU output)
    auto group_sums = [&](int rbase) {
        const int rl = tid >> 2, gi = (tid >> 1) & 1, hf = tid & 1;
        float sum = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 v = *reinterpret_cast<const uint4*>(&tile[rl * TS + gi * 64 + hf * 32 + c * 8]);
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                sum += bf16_to_f32(w4[q] & 0xffffu);
                sum += bf16_to_f32(w4[q] >> 16);
            }
        }
        const float other = __shfl_xor(sum, 1);
        if (hf == 0 && m0 + rbase + rl < M)
            p.ysum[(int64_t)((n0 >> 6) + gi) * M + m0 + rbase + rl] = sum + other;
    };
    if (paired_out) {
        static_assert(kThreads == 4 * 64, "four threads per tile row");
        __syncthreads();                                           // every wave is done with the stages
        emit(0, 0);
        emit(1, 0);
        __syncthreads();
        group_sums(0);
        __syncthreads();                                           // the tile is read before rows 64-127
        emit(2, 64);
        emit(3, 64);
        __syncthreads();
        group_sums(64);
    } else {
        emit(0, 0);
        emit(1, 0);
        emit(2, 0);
        emit(3, 0);
    }
}

// ---------------------------------------------------------------------------
// Activation pre-pass: one wave per row.  Pass 1 forms the row's sum of
// squares (with the norm; the per-element formula of mq4_rms_norm) and the
// largest |x (1 + w)| (|x| without the norm); pass 2 writes bf16(x r (1 + w))
// (or x), scaled by 2^-e and converted to fp16, in the pair order, and
// xscale[m] = 2^e.  e is the smallest such that the scaled row stays below
// 2^15 (0 for every normalized row whose values stay below 2^15).  With CAP >
// 0 (K <= 512 CAP) a lane keeps its chunks of x and of the norm weight in
// registers between the passes (all loads issued first), so the row is read
// once; the sums keep the chunk order of the reloading form (CAP = 0).  With
// lut, the blocks past the rows' write the SiLU table (silu_lut_entry), one
// entry per thread.
template <bool NORM, int CAP>
__global__ __launch_bounds__(256) void pair_rows16_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                          const uint16_t* __restrict__ nw, float eps,
                                                          uint16_t* __restrict__ xp, float* __restrict__ xscale,
                                                          uint16_t* __restrict__ lut) {
#pragma clang fp contract(off)
    const int row_blocks = (M + 3) / 4;
    if ((int)blockIdx.x >= row_blocks) {
        const uint32_t i = (blockIdx.x - (uint32_t)row_blocks) * 256u + threadIdx.x;
        if (i < (uint32_t)SILU_LUT_N) lut[i] = (uint16_t)silu_lut_entry(i);
        return;
    }
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;                                  // whole waves
    const int CH = K / 8;
    const uint4* src = reinterpret_cast<const uint4*>(x + (int64_t)m * K);
    const uint4* nw4 = reinterpret_cast<const uint4*>(nw);
    uint4* dst = reinterpret_cast<uint4*>(xp + (int64_t)m * K);
    constexpr int NC = CAP > 0 ? CAP : 1;
    uint4 xc[NC], wc[NC];
    if (CAP > 0) {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lane + 64 * i;
            if (c < CH) {
                xc[i] = src[c];
                wc[i] = NORM ? nw4[c] : make_uint4(0, 0, 0, 0);
            }
        }
    }
    float ss = 0.0f, big = 0.0f;
    auto scan = [&](const uint4& v, const uint4& wv) {
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
        const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (NORM) ss = sumsq_word(ss, vw[q]);
            const float a0 = bf16_to_f32(vw[q] & 0xffffu), a1 = bf16_to_f32(vw[q] >> 16);
            const float f0 = NORM ? 1.0f + bf16_to_f32(ww[q] & 0xffffu) : 1.0f;
            const float f1 = NORM ? 1.0f + bf16_to_f32(ww[q] >> 16) : 1.0f;
            big = fmaxf(big, fmaxf(fabsf(a0 * f0), fabsf(a1 * f1)));
        }
    };
    if (CAP > 0) {
#pragma unroll
        for (int i = 0; i < NC; ++i)
            if (lane + 64 * i < CH) scan(xc[i], wc[i]);
    } else {
        for (int c = lane; c < CH; c += 64) scan(src[c], NORM ? nw4[c] : make_uint4(0, 0, 0, 0));
    }
    float r = 1.0f;
    if (NORM) r = rms_inv(wave_sum(ss), K, eps);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) big = fmaxf(big, __shfl_xor(big, off));
    big *= NORM ? r : 1.0f;
    // the largest output is below big * (1 + 2^-8) (one bf16 rounding)
    int e = 0;
    while (!(big * 1.01f < 32768.0f * __builtin_ldexpf(1.0f, e)) && e < 200) ++e;
    const float down = __builtin_ldexpf(1.0f, -e);
    if (lane == 0) xscale[m] = __builtin_ldexpf(1.0f, e);
    auto emit = [&](int c, uint4 v, const uint4& w) {
        if (NORM)
            v = make_uint4(norm_word(v.x, w.x, r), norm_word(v.y, w.y, r), norm_word(v.z, w.z, r),
                           norm_word(v.w, w.w, r));
        uint32_t pr[4];
        pair_chunk(v, pr, 0.0f);
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const h2_t hv = {(_Float16)(bf16_to_f32(pr[q] & 0xffffu) * down),
                             (_Float16)(bf16_to_f32(pr[q] >> 16) * down)};
            o[q] = __builtin_bit_cast(uint32_t, hv);
        }
        dst[c] = make_uint4(o[0], o[1], o[2], o[3]);
    };
    if (CAP > 0) {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lane + 64 * i;
            if (c < CH) emit(c, xc[i], wc[i]);
        }
    } else {
        for (int c = lane; c < CH; c += 64) emit(c, src[c], NORM ? nw4[c] : make_uint4(0, 0, 0, 0));
    }
}

// y = bf16(res + round_bf16(part[0] + part[1] + ... + part[S - 1])), the
// parts added in order: 4 elements per thread (MN % 4 == 0, 16-byte aligned
// parts, 8-byte aligned res and y), S <= 4.
__global__ __launch_bounds__(256) void kpart_residual_kernel(const float* __restrict__ part, int S, int64_t MN,
                                                             const uint16_t* __restrict__ res,
                                                             uint16_t* __restrict__ y) {
#pragma clang fp contract(off)
    const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (e >= MN) return;
    // every load issued before the first add (S <= 4 parts)
    float4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (k < S) v[k] = *reinterpret_cast<const float4*>(part + (int64_t)k * MN + e);
    const uint2 r = *reinterpret_cast<const uint2*>(res + e);
    float4 sum = v[0];
#pragma unroll
    for (int k = 1; k < 4; ++k) {
        if (k < S) {
            sum.x += v[k].x;
            sum.y += v[k].y;
            sum.z += v[k].z;
            sum.w += v[k].w;
        }
    }
    const float sv[4] = {sum.x, sum.y, sum.z, sum.w};
    const uint32_t rv[4] = {r.x & 0xffffu, r.x >> 16, r.y & 0xffffu, r.y >> 16};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = f32_to_bf16(bf16_to_f32(rv[q]) + round_bf16(sv[q]));
    *reinterpret_cast<uint2*>(y + e) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
}

}  // namespace g16

int launch_pair_rows16(const uint16_t* x, int M, int K, const uint16_t* norm_w, float eps, uint16_t* xp,
                       float* xscale, uint16_t* silu_lut, hipStream_t st) {
    if (M < 1 || K % 512 != 0) return -1;
    const unsigned blocks = (unsigned)((M + 3) / 4) + (silu_lut ? (unsigned)(SILU_LUT_N / 256) : 0u);
    // rows of at most 4 chunks per lane (K <= 2048) read once
    const bool cached = K / 512 <= 4;
    if (norm_w && cached)
        hipLaunchKernelGGL((g16::pair_rows16_kernel<true, 4>), dim3(blocks), dim3(256), 0, st, x, M, K, norm_w, eps,
                           xp, xscale, silu_lut);
    else if (norm_w)
        hipLaunchKernelGGL((g16::pair_rows16_kernel<true, 0>), dim3(blocks), dim3(256), 0, st, x, M, K, norm_w, eps,
                           xp, xscale, silu_lut);
    else if (cached)
        hipLaunchKernelGGL((g16::pair_rows16_kernel<false, 4>), dim3(blocks), dim3(256), 0, st, x, M, K, norm_w, eps,
                           xp, xscale, silu_lut);
    else
        hipLaunchKernelGGL((g16::pair_rows16_kernel<false, 0>), dim3(blocks), dim3(256), 0, st, x, M, K, norm_w, eps,
                           xp, xscale, silu_lut);
    return 0;
}

int launch_q4_gemm16(const Gemm16Args& a, int epi, hipStream_t st) {
    // 32-bit byte offsets in the kernel; whole blocks of 8 groups (K % 512,
    // the scale/bias DMA) with scale/bias rows 16-byte aligned
    const bool fits32 = (int64_t)a.M * a.K * 2 <= 0xFFFFFFFFLL && (int64_t)a.N * a.K / 2 <= 0xFFFFFFFFLL;
    auto a16 = [](const QMat& q) { return reinterpret_cast<uintptr_t>(q.s) % 16 == 0 && reinterpret_cast<uintptr_t>(q.b) % 16 == 0; };
    if (!fits32 || a.K % 512 != 0 || a.M < 1 || a.N < 1 || !a16(a.A) || (epi == GEMM_SWIGLU && !a16(a.B))) return -1;
    if (a.ysum && (epi != GEMM_SWIGLU || a.yscale != 0.0f || a.N % 128 != 0)) return -1;
    if (a.yscale != 0.0f && (epi != GEMM_SWIGLU || a.N % 8 != 0)) return -1;
    if (epi == GEMM_SWIGLU && (!a.silu_lut || !aligned(a.silu_lut, 16))) return -1;
    // K parts: GEMM_RESIDUAL only, at most 4, whole 8-group scale slots per
    // part, fp32 parts [ksplit][M][N] (16-byte aligned, N % 4 == 0) combined
    // by a second kernel
    const int S = a.ksplit > 1 ? a.ksplit : 1;
    if (S > 1 && (epi != GEMM_RESIDUAL || S > 4 || (a.K / 64) % (8 * S) != 0 || !a.part ||
                  reinterpret_cast<uintptr_t>(a.part) % 16 != 0 || a.N % 4 != 0 || !aligned(a.res, 8) ||
                  !aligned(a.y, 8)))
        return -1;
    // 128-column tiles (three blocks per CU) for the residual product when
    // asked for, else 256
    const bool narrow = epi == GEMM_RESIDUAL && a.narrow;
    const int BN = epi == GEMM_SWIGLU ? g16::Cols<2>::BNW / 2 : narrow ? g16::Cols<1>::BNW : g16::Cols<2>::BNW;
    const unsigned blocks = (unsigned)(((a.N + BN - 1) / BN) * ((a.M + g16::TBM - 1) / g16::TBM) * S);
    switch (epi) {
        case GEMM_RESIDUAL: {
            if (narrow)
                hipLaunchKernelGGL((g16::q4_gemm16_kernel<GEMM_RESIDUAL, 1>), dim3(blocks), dim3(g16::kThreads), 0, st,
                                   a);
            else
                hipLaunchKernelGGL((g16::q4_gemm16_kernel<GEMM_RESIDUAL, 2>), dim3(blocks), dim3(g16::kThreads), 0, st,
                                   a);
            if (S > 1) {
                const int64_t MN = (int64_t)a.M * a.N;
                hipLaunchKernelGGL(g16::kpart_residual_kernel, dim3((unsigned)((MN / 4 + 255) / 256)), dim3(256), 0,
                                   st, a.part, S, MN, a.res, reinterpret_cast<uint16_t*>(a.y));
            }
            return 0;
        }
        case GEMM_SWIGLU:
            hipLaunchKernelGGL((g16::q4_gemm16_kernel<GEMM_SWIGLU, 2>), dim3(blocks), dim3(g16::kThreads), 0, st, a);
            return 0;
        default:
            return -1;
    }
}

}  // namespace mq4
