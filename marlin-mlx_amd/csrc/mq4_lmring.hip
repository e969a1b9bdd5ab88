// Batched lm_head + argmax with a weight ring, gfx950: for M token rows
// (1 <= M <= 32) at K = 2048,
//
//   logits = lm_head(rms_norm(x, w)),   idx[m] = argmax(logits[m])
//
// (src/model/marlin.cpp:145, 161-169; src/sampling/sampler.cpp:14-16) with
// exactly the arithmetic of the MFMA GEMV's argmax epilogue in mq4_mfma.hip:
// K split over 8 waves of 4 groups each, the per-group fold
// acc = s * P' + (c * X + acc) on exact bf16 x (128 + q) MFMA products, the
// wave partials summed in wave order, one bf16 rounding per logit, the
// (bf16 key, lowest index) argmax.  Logits and tokens are bit-identical to it.
//
// What differs is the weight stream.  One persistent 8-wave workgroup per CU
// walks the 16-row tiles blockIdx.x, blockIdx.x + gridDim.x, ...; each wave
// keeps kR tiles of its 128-byte line per row in flight, staged into LDS by
// DMA as whole lines (about 100 KB per CU in flight, the bytes the HBM
// latency needs), where the GEMV holds one tile in registers.  Per tile the
// eight wave partials meet in LDS (double-buffered, one barrier per tile)
// and wave (tile % 8) sums them, rounds and updates its running argmax.
#include "mq4_device.h"
#include "mq4_gemv.h"
#include "mq4_host.h"
#include "mq4_mfma_ops.h"
#include "mq4_stage.h"

namespace mq4 {
namespace lmr {

using stage::dma16;
using stage::dma4;
using stage::stage_chunk;
using stage::stage_slot;

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int K = 2048;
constexpr int GA = K / 64;            // groups per row (32)
constexpr int GWA = GA / kWaves;      // groups per wave (4)
constexpr int kR = 6;                 // tiles in flight per wave
constexpr int kDmaPerTile = 3;        // two 1 KB line blocks + one scale/bias block
constexpr int kMaxM = 32;

struct Params {
    const uint16_t* x;         // [M, K] bf16
    const uint16_t* norm;      // [K] (1 + w) RMSNorm weight (NORM)
    float eps;
    QMat A;                    // [N, K] Q4
    int M, N;
    uint16_t* y;               // [M, N] bf16 logits, or null
    uint64_t* partial;         // [M][kPartialStride] per-workgroup best keys
};

struct alignas(16) Smem {
    uint4 w[kWaves][kR][2][64];            // each wave's line blocks, rows 0-7 and 8-15 (96 KB)
    uint32_t sb[kWaves][kR][64];           // each wave's scales (dwords 0-31) and biases (32-63)
    mf::f32x4_t red[2][kWaves][2][64];     // wave partials, double-buffered by tile parity
    float ss[kWaves][kMaxM];
    uint64_t best[kWaves][kMaxM];
};

template <int N>
__device__ __forceinline__ void wait_tiles_after(int n) {
    // at most n later tiles (kDmaPerTile DMA each) may stay in flight
    static_assert(N == kR - 1, "ring depth");
    switch (n) {
        case 5: wait_vmcnt<5 * kDmaPerTile>(); break;
        case 4: wait_vmcnt<4 * kDmaPerTile>(); break;
        case 3: wait_vmcnt<3 * kDmaPerTile>(); break;
        case 2: wait_vmcnt<2 * kDmaPerTile>(); break;
        case 1: wait_vmcnt<1 * kDmaPerTile>(); break;
        default: wait_vmcnt<0>(); break;
    }
}

template <int MT, bool NORM>
__global__ __launch_bounds__(kThreads) void lm_ring_kernel(Params p) {
#pragma clang fp contract(off)
    __shared__ Smem sm;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c16 = lane & 15, kq = lane >> 4;
    const int M = p.M, N = p.N, g0 = wave * GWA;
    // Rows in R full rounds of 16-row tiles (tile j of workgroup b: rows
    // 16 (b + j G) ..), and the remaining rem < 16 G rows as one short tile
    // of at most q = ceil(rem / G) rows per workgroup, taken first: its
    // round trip then overlaps the ring's start instead of adding a last
    // round on a fraction of the CUs.  A short tile's missing rows repeat
    // its last row and are not reported.
    const int G = (int)gridDim.x, bx = (int)blockIdx.x;
    const int R = N / (16 * G), rem = N - R * 16 * G;
    const int q = (rem + G - 1) / G;
    const int rshort = R * 16 * G + bx * q;
    const int nshort = rem == 0 ? 0 : (N - rshort < q ? (N - rshort > 0 ? N - rshort : 0) : q);
    const int S = nshort > 0 ? 1 : 0;
    const int T = R + S;
    auto tile_n0 = [&](int j) { return j < S ? rshort : 16 * (bx + (j - S) * G); };
    auto tile_rows = [&](int j) { return j < S ? nshort : 16; };

    // ---- activations and norm weights (tracked loads, waited for before any DMA) ----
    uint4 xa[MT][GWA][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + c16;
        const int mm = m < M ? m : M - 1;              // rows >= M repeat row M - 1, never read back
#pragma unroll
        for (int gi = 0; gi < GWA; ++gi) {
            const uint4* src = reinterpret_cast<const uint4*>(p.x + (int64_t)mm * K + 64 * (g0 + gi) + 16 * kq);
            xa[mt][gi][0] = src[0];
            xa[mt][gi][1] = src[1];
        }
    }
    uint4 nwv[GWA][2];
    if constexpr (NORM) {
#pragma unroll
        for (int gi = 0; gi < GWA; ++gi) {
            const uint4* src = reinterpret_cast<const uint4*>(p.norm + 64 * (g0 + gi) + 16 * kq);
            nwv[gi][0] = src[0];
            nwv[gi][1] = src[1];
        }
        // sums of squares: this lane's 16 values per group, the four k blocks
        // of the wave, then the 8 waves in wave order (as the MFMA GEMV)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            float s = 0.0f;
#pragma unroll
            for (int gi = 0; gi < GWA; ++gi) {
                mf::sumsq4(s, xa[mt][gi][0]);
                mf::sumsq4(s, xa[mt][gi][1]);
            }
            s += __shfl_xor(s, 16);
            s += __shfl_xor(s, 32);
            if (kq == 0) sm.ss[wave][16 * mt + c16] = s;
        }
    }
    wait_vmcnt<0>();

    // ---- the ring: tile j of this workgroup -> slot j % kR ----
    auto issue = [&](int j, int slot) {
        const int n0 = tile_n0(j), nl = n0 + tile_rows(j) - 1;  // rows past nl repeat row nl, never used
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int sl = 64 * b + lane, row = sl >> 3, u = stage_chunk(sl, row);
            const int n = n0 + row < nl ? n0 + row : nl;
            dma16(p.A.wq + (int64_t)n * (K / 8) + 32 * wave + 4 * u, &sm.w[wave][slot][b][0]);
        }
        const int r = (lane & 31) >> 1, n = n0 + r < nl ? n0 + r : nl;
        const uint16_t* src = lane < 32 ? p.A.s : p.A.b;
        dma4(src + (int64_t)n * GA + GWA * wave + 2 * (lane & 1), &sm.sb[wave][slot][0]);
    };
#pragma unroll
    for (int j = 0; j < kR; ++j)
        if (j < T) issue(j, j);
    lds_barrier();                                     // sums of squares

    // ---- normalized, pair-ordered activations and their group sums ----
    const uint4 ones = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
    const mf::f32x4_t zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    mf::f32x4_t X[MT][GWA];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if constexpr (NORM) {
            float tot = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) tot += sm.ss[w][16 * mt + c16];
            const float r = rms_inv(tot, K, p.eps);
#pragma unroll
            for (int gi = 0; gi < GWA; ++gi)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint4 v = xa[mt][gi][h], w = nwv[gi][h];
                    xa[mt][gi][h] = make_uint4(norm_word(v.x, w.x, r), norm_word(v.y, w.y, r), norm_word(v.z, w.z, r),
                                               norm_word(v.w, w.w, r));
                }
        }
#pragma unroll
        for (int gi = 0; gi < GWA; ++gi) {
            xa[mt][gi][0] = mf::pair_order(xa[mt][gi][0]);
            xa[mt][gi][1] = mf::pair_order(xa[mt][gi][1]);
            X[mt][gi] = mf::mfma16(xa[mt][gi][1], ones, mf::mfma16(xa[mt][gi][0], ones, zero4));
        }
    }

    // Each tile's 16 x 16 MT outputs are summed by all eight waves, 32 MT
    // each: thread t of wave v takes output i = t % 4 of partial lane
    // l = 8 v + (t % 32) / 4 of tile mt = t / 32, i.e. row
    // m = 16 mt + 4 (v / 2) + i of column c = l % 16 (fixed across tiles).
    const bool red_on = lane < 32 * MT;
    const int r_mt = lane >> 5, r_l = 8 * wave + ((lane & 31) >> 2), r_i = lane & 3;
    const int r_m = 16 * r_mt + 4 * (r_l >> 4) + r_i, r_c = r_l & 15;
    uint64_t best = 0;

    for (int j = 0; j < T; ++j) {
        const int slot = j % kR;
        wait_tiles_after<kR - 1>(T - 1 - j < kR - 1 ? T - 1 - j : kR - 1);
        mf::f32x4_t acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = zero4;
        const uint2* wl = reinterpret_cast<const uint2*>(&sm.w[wave][slot][0][0]);
        const uint32_t* sbl = &sm.sb[wave][slot][0];
#pragma unroll
        for (int gi = 0; gi < GWA; ++gi) {
            const uint2 wv = wl[2 * stage_slot(c16, c16, 2 * gi + (kq >> 1)) + (kq & 1)];
            const uint4 b0 = mf::unpack_word(wv.x), b1 = mf::unpack_word(wv.y);
            const uint32_t sw = sbl[2 * c16 + (gi >> 1)], bw = sbl[32 + 2 * c16 + (gi >> 1)];
            const float s = bf16_to_f32((gi & 1) ? (sw >> 16) : (sw & 0xffffu));
            const float c = affine_c(s, (gi & 1) ? (bw >> 16) : (bw & 0xffffu));
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const mf::f32x4_t P = mf::mfma16(xa[mt][gi][1], b1, mf::mfma16(xa[mt][gi][0], b0, zero4));
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[mt][i] = __builtin_fmaf(s, P[i], __builtin_fmaf(c, X[mt][gi][i], acc[mt][i]));
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) sm.red[j & 1][wave][mt][lane] = acc[mt];
        lds_barrier();                                 // this tile's partials; this wave's slot reads done
        if (j + kR < T) issue(j + kR, slot);
        if (red_on) {
            // the 8 partials in wave order, one bf16 rounding, the running argmax
            const float* rp = reinterpret_cast<const float*>(&sm.red[j & 1][0][r_mt][r_l]) + r_i;
            constexpr int kStride = 2 * 64 * 4;            // floats from one wave's partials to the next
            float v = rp[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) v += rp[w * kStride];
            const int n = tile_n0(j) + r_c;
            if (r_m < M && r_c < tile_rows(j)) {
                const uint32_t lb = f32_to_bf16(v);
                if (p.y) p.y[(int64_t)r_m * N + n] = (uint16_t)lb;
                const uint64_t key = argmax_key(lb, (uint32_t)n);
                best = key > best ? key : best;
            }
        }
    }

    // ---- per-workgroup best key of each row: the 8 columns of a wave's
    // threads (t = 32 mt + 4 a + i, a = 0..7), then the two waves v, v ^ 1 ----
    uint64_t b = best;
#pragma unroll
    for (int off = 4; off < 32; off <<= 1) {
        const uint64_t o = shfl_xor_u64(b, off);
        b = o > b ? o : b;
    }
    if (red_on && (lane & 28) == 0) sm.best[wave][r_m] = b;
    __syncthreads();
    if (tid < M) {
        // rows 16 mt + 4 (v / 2) + i are held by waves v = 2 (m % 16 / 4) and v + 1
        const int v0 = 2 * ((tid & 15) >> 2);
        const uint64_t b0 = sm.best[v0][tid], b1 = sm.best[v0 + 1][tid];
        p.partial[(int64_t)tid * kPartialStride + blockIdx.x] = b1 > b0 ? b1 : b0;
    }
}

}  // namespace lmr

// ---- 1-2 rows: the dot2 GEMV's arithmetic through the same kind of ring ----
//
// The dot2 GEMV (mq4_gemv.hip, K = 2048: one 16-byte slice per lane, 4 rows
// per iteration, no K split) forms each logit as: per lane, the dot2 chain
// of its slice's 4 words, the group fold s * D + c * X added to 0, then
// wave_multi_reduce over the 64 lanes.  This kernel forms every logit the
// same way (so logits and tokens are bit-identical to it, and the one-launch
// decode step, which reproduces the dot2 GEMV, keeps its token) but feeds it
// differently: each of 16 waves per CU streams its own 4-row batches with
// two batches in flight, a 1 KB row per DMA instruction (lane l receives
// slice l), and the four rows' scales and biases as two contiguous 256-byte
// runs.  Every DMA takes a scalar base and a constant per-lane offset, so no
// vector instruction goes to addressing; the waves meet only at the end.
namespace lmd {

constexpr int kWaves = 16;
constexpr int kThreads = 64 * kWaves;
constexpr int K = 2048;
constexpr int RPI = 4;                 // rows per batch (the dot2 GEMV's)
constexpr int kRD = 2;                 // batches in flight per wave
constexpr int kDmaPerBatch = RPI + 2;

struct alignas(16) Smem {
    uint4 w[kWaves][kRD][RPI][64];     // row r of a batch: lane l's slice l (128 KB)
    uint32_t sb[kWaves][kRD][2][64];   // scales, then biases, of the 4 rows (16 dwords per row)
    uint64_t best[kWaves][2];
};

template <int M, bool NORM>
__global__ __launch_bounds__(kThreads) void lm_ring_dot2_kernel(lmr::Params p) {
#pragma clang fp contract(off)
    constexpr int V = RPI * M;
    constexpr int SH = 6 - log2_const<V>();
    __shared__ Smem sm;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Rows in R full rounds of RPI-row batches (batch j of wave gw: rows
    // RPI (gw + j W) ..), then the remaining rem < RPI W rows as one short
    // batch of at most q = ceil(rem / W) rows per wave, dealt wave-major
    // (wave v of every workgroup before wave v + 1 of any), so that every
    // CU ends within a few rows of the others: a last round of whole batches
    // on a fraction of the CUs cost 1.2-1.6 us at N = 248320.  A short
    // batch's missing rows get a 256-byte DMA of its last row instead (the
    // same DMA count per batch, a quarter of the bytes) and are not reported.
    const int N = p.N;
    const int gw = (int)blockIdx.x * kWaves + wave, W = (int)gridDim.x * kWaves;
    const int R = N / (RPI * W), rem = N - R * RPI * W;
    const int q = (rem + W - 1) / W;
    const int rlast = R * RPI * W + (wave * (int)gridDim.x + (int)blockIdx.x) * q;   // short batch
    const int nlast = rem == 0 ? 0 : (N - rlast < q ? (N - rlast > 0 ? N - rlast : 0) : q);
    const int S = nlast > 0 ? 1 : 0;                           // the short batch goes first
    const int T = R + S;
    auto first_row = [&](int j) { return j < S ? rlast : RPI * (gw + (j - S) * W); };
    auto batch_rows = [&](int j) { return j < S ? nlast : RPI; };
    const char* wq = reinterpret_cast<const char*>(p.A.wq);
    const char* sq = reinterpret_cast<const char*>(p.A.s);
    const char* bq = reinterpret_cast<const char*>(p.A.b);

    auto issue = [&](int j, int slot) {
        const int64_t r0 = first_row(j);
        const int nr = batch_rows(j);
#pragma unroll
        for (int r = 0; r < RPI; ++r) {
            if (r < nr)
                stage::dma16_s(wq + (r0 + r) * (K / 2), 16u * lane, &sm.w[wave][slot][r][0]);
            else
                stage::dma4_s(wq + (r0 + nr - 1) * (K / 2), 4u * lane, &sm.w[wave][slot][r][0]);
        }
        // scales and biases: lane l holds dword l % 16 of row l / 16
        const uint32_t sbo = 64u * (uint32_t)((lane >> 4) < nr ? (lane >> 4) : nr - 1) + 4u * (lane & 15);
        stage::dma4_s(sq + r0 * (K / 32), sbo, &sm.sb[wave][slot][0][0]);
        stage::dma4_s(bq + r0 * (K / 32), sbo, &sm.sb[wave][slot][1][0]);
    };
#pragma unroll
    for (int j = 0; j < kRD; ++j)
        if (j < T) issue(j, j);

    // ---- this lane's slice of the activations (tracked loads issued after
    // the DMA: loads complete in issue order, so they arrive with it) ----
    uint4 xv[M][4];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int w = 0; w < 4; ++w) xv[m][w] = reinterpret_cast<const uint4*>(p.x + (int64_t)m * K)[lane * 4 + w];
    if constexpr (NORM) {
        uint4 wn[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) wn[w] = reinterpret_cast<const uint4*>(p.norm)[lane * 4 + w];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint4 a = xv[m][w];
                s = sumsq_word(s, a.x);
                s = sumsq_word(s, a.y);
                s = sumsq_word(s, a.z);
                s = sumsq_word(s, a.w);
            }
            const float r = rms_inv(wave_sum(s), K, p.eps);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint4 e = xv[m][w];
                xv[m][w] = make_uint4(norm_word(e.x, wn[w].x, r), norm_word(e.y, wn[w].y, r),
                                      norm_word(e.z, wn[w].z, r), norm_word(e.w, wn[w].w, r));
            }
        }
    }
    uint32_t xp[M][16];
    float xs[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) sum = pair_chunk(xv[m][w], &xp[m][4 * w], sum);
        xs[m] = sum;
    }

    uint64_t best = 0;
    const int sbw = lane >> 2, sbh = (lane >> 1) & 1;  // dword and half of this slice's group (lane / 2)
    for (int j = 0; j < T; ++j) {
        const int slot = j % kRD;
        static_assert(kRD == 2, "one later batch may stay in flight");
        if (j + 1 < T) wait_vmcnt<kDmaPerBatch>();
        else wait_vmcnt<0>();
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int r = 0; r < RPI; ++r) {
            const uint4 wv = sm.w[wave][slot][r][lane];
            const uint32_t sw = sm.sb[wave][slot][0][16 * r + sbw], bw = sm.sb[wave][slot][1][16 * r + sbw];
            const uint32_t sbits = sbh ? (sw >> 16) : (sw & 0xffffu), bbits = sbh ? (bw >> 16) : (bw & 0xffffu);
            float d[M];
#pragma unroll
            for (int m = 0; m < M; ++m) d[m] = 0.0f;
            const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t p0 = nib_pair_bf16<0>(wd[w]);
                const uint32_t p1 = nib_pair_bf16<1>(wd[w]);
                const uint32_t p2 = nib_pair_bf16<2>(wd[w]);
                const uint32_t p3 = nib_pair_bf16<3>(wd[w]);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    d[m] = dot2_bf16(xp[m][4 * w + 0], p0, d[m]);
                    d[m] = dot2_bf16(xp[m][4 * w + 1], p1, d[m]);
                    d[m] = dot2_bf16(xp[m][4 * w + 2], p2, d[m]);
                    d[m] = dot2_bf16(xp[m][4 * w + 3], p3, d[m]);
                }
            }
#pragma unroll
            for (int m = 0; m < M; ++m) acc[r * M + m] += affine_term(sbits, bbits, d[m], xs[m]);
        }
        // every read of this slot is done before its refill is issued
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (j + kRD < T) issue(j + kRD, slot);
        const float val = wave_multi_reduce<V>(acc, lane);
        const int vidx = lane >> SH, m = vidx % M, row = first_row(j) + vidx / M;
        if ((lane & ((1 << SH) - 1)) == 0 && m < p.M && vidx / M < batch_rows(j)) {
            const uint32_t lb = f32_to_bf16(val);
            if (p.y) p.y[(int64_t)m * N + row] = (uint16_t)lb;
            const uint64_t key = argmax_key(lb, (uint32_t)row);
            best = key > best ? key : best;
        }
    }
    // ---- per-workgroup best key of each row: lanes of the same m (lane bit
    // SH holds m for M = 2), then the waves ----
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        if (M == 2 && off == (1 << SH)) continue;
        const uint64_t o = shfl_xor_u64(best, off);
        best = o > best ? o : best;
    }
    if (lane < (M << SH) && (lane & ((1 << SH) - 1)) == 0) sm.best[wave][lane >> SH] = best;
    __syncthreads();
    if (tid < p.M) {
        uint64_t b = sm.best[0][tid];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) b = sm.best[w][tid] > b ? sm.best[w][tid] : b;
        p.partial[(int64_t)tid * kPartialStride + blockIdx.x] = b;
    }
}

}  // namespace lmd

int launch_lm_ring(const GemvParams& a, bool norm, hipStream_t st) {
    if (a.K != lmr::K || a.m_valid < 1 || a.m_valid > lmr::kMaxM || a.N < 1 || !a.partial || !a.idx) return -1;
    if (!aligned(a.x, 16) || !aligned(a.A.wq, 16) || !aligned(a.A.s, 4) || !aligned(a.A.b, 4)) return -1;
    if (norm && !aligned(a.norm_w, 16)) return -1;
    const int ntiles = (a.N + 15) / 16;
    int grid = num_cus();
    if (grid > ntiles) grid = ntiles;
    if (grid > kPartialStride) grid = kPartialStride;
    lmr::Params p{};
    p.x = a.x;
    p.norm = a.norm_w;
    p.eps = a.eps;
    p.A = a.A;
    p.M = a.m_valid;
    p.N = a.N;
    p.y = a.y;
    p.partial = a.partial;
    const dim3 g((unsigned)grid), b(lmr::kThreads);
    if (a.m_valid <= 2) {
        const dim3 bd(lmd::kThreads);
        if (a.m_valid == 1) {
            if (norm) hipLaunchKernelGGL((lmd::lm_ring_dot2_kernel<1, true>), g, bd, 0, st, p);
            else hipLaunchKernelGGL((lmd::lm_ring_dot2_kernel<1, false>), g, bd, 0, st, p);
        } else {
            if (norm) hipLaunchKernelGGL((lmd::lm_ring_dot2_kernel<2, true>), g, bd, 0, st, p);
            else hipLaunchKernelGGL((lmd::lm_ring_dot2_kernel<2, false>), g, bd, 0, st, p);
        }
    } else if (a.m_valid <= 16) {
        if (norm) hipLaunchKernelGGL((lmr::lm_ring_kernel<1, true>), g, b, 0, st, p);
        else hipLaunchKernelGGL((lmr::lm_ring_kernel<1, false>), g, b, 0, st, p);
    } else {
        if (norm) hipLaunchKernelGGL((lmr::lm_ring_kernel<2, true>), g, b, 0, st, p);
        else hipLaunchKernelGGL((lmr::lm_ring_kernel<2, false>), g, b, 0, st, p);
    }
    launch_argmax_finalize(a.partial, grid, a.m_valid, a.idx, st);
    return 0;
}

}  // namespace mq4
