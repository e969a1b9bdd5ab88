// One launch per MLP half for a batch of M token rows (1 <= M <= 32), gfx950:
//
//   x_out = x + down(swiglu(gate n, up n)),   n = rms_norm(x, norm)
//
// i.e. src/model/marlin.cpp:141-142 (rms_norm :12-16, mlp_forward :31-35,
// residual add) for M concurrent decode streams (src/core/engine.cpp:79-94),
// with the per-element arithmetic of the MFMA GEMV (mq4_mfma.hip): exact
// bf16 x (128 + q) products on v_mfma_f32_16x16x32_bf16, fp32 sums, the fold
// acc = s * P' + (c * X + acc) per group, the (1 + w) RMSNorm and the bf16
// SwiGLU / residual of mq4_device.h.
//
// Why one launch: the MFMA GEMV path runs the layer as three launches
// (gate/up + SwiGLU, the down product in two K parts, their combine), each a
// 7-14 MB pass paying its own dispatch, ramp-up and HBM latency (27 us per
// layer at M = 16 for 21 MB of weights).  Here every workgroup issues all of
// its weights (83 KB) and its activations at the start, and the workgroups
// meet twice inside the launch:
//
// Work split by XCD (workgroup w runs on XCD w % 8, rank r = w / 8; only the
// speed depends on that placement, every exchanged word is written and read
// at device scope):
//   gate/up: XCD j owns rows [768 j, 768 j + 768) of both matrices;
//     workgroup (j, r) rows 768 j + 24 r + [0, 24), as three 16-row MFMA
//     tiles of [its 24 gate rows; its 24 up rows], K split over its 8 waves
//     (4 groups each), the wave partials added in wave order;
//   h exchange inside the XCD: each workgroup publishes its M x 24 h values;
//     every workgroup of XCD j gathers the XCD's M x 768 slice of h;
//   down: workgroup (j, r) multiplies that slice with columns [768 j,
//     768 j + 768) of down rows [64 r, 64 r + 64): 4 tiles x 12 groups, two
//     waves per tile (6 groups each), added wave-pair-wise in order;
//   part sums across XCDs: workgroup (j, r) publishes its M x 64 part-j sums
//     and reads, for its 8 rows [64 r + 8 j, 64 r + 8 j + 8), the part sums
//     of the same rows from the seven other XCDs; it adds the eight parts in
//     part order, then the residual, and writes those 8 rows of x_out.
//
// Words travel as 64-bit tagged words (two bf16 or one fp32 in the low half,
// a 32-bit tag in the high half), self-validating, written once per launch.
// The tag base comes from an epoch word in the workspace (zero-filled once):
// every workgroup reads it, then counts itself in with one atomic add, and
// the one that completes the count of 256 (all have read the epoch) stores
// epoch + 1 for the next launch.  Every wait is bounded: on a timeout a sticky
// error word is set, every workgroup writes NaN into its rows of x_out and
// leaves, and later launches with that workspace do the same until it is
// zero-filled again.
#include "mq4_device.h"
#include "mq4_host.h"
#include "mq4_mfma_ops.h"
#include "mq4_stage.h"

#include <mutex>

namespace mq4 {

namespace rows {

using stage::dma16;
using stage::dma4;
using stage::stage_chunk;
using stage::stage_slot;

constexpr int kNWG = 256;            // workgroups (one per CU)
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kXcd = 8;
constexpr int kRanks = kNWG / kXcd;  // 32
constexpr int H = 2048;              // hidden size this instance is built for
constexpr int I = 6144;              // intermediate size
constexpr int IX = I / kXcd;         // 768: h slice / down K part of one XCD
constexpr int GA = H / 64;           // gate/up groups (32)
constexpr int GWA = GA / kWaves;     // gate/up groups per wave (4)
constexpr int RA = IX / kRanks;      // gate (and up) rows per workgroup (24)
constexpr int NTA = 2 * RA / 16;     // gate/up MFMA tiles (3)
constexpr int RB = H / kRanks;       // down rows per workgroup (64)
constexpr int NTB = RB / 16;         // down tiles (4)
constexpr int GB = IX / 64;          // down groups per part (12)
constexpr int GWB = GB * NTB / kWaves;  // down groups per wave (6)
constexpr int ROUT = RB / kXcd;      // x rows each workgroup sums and writes (8)
constexpr int kMaxM = 32;
constexpr int HWD = IX / 2;          // h words of one row of an XCD's slice (384)
constexpr int HLD = HWD + 4;         // LDS row stride of the slice (16 rows read at once hit 16 bank groups)
constexpr int MP = kMaxM + 1;        // LDS row stride of the [row][m] sums
constexpr int kSleep0 = 16;          // s_sleep units (64 clocks) before a first poll round
static_assert(NTA * 16 == 2 * RA && GWB * kWaves == GB * NTB && GWB * 2 == GB, "tiling");

struct Params {
    const uint16_t* x;         // [M, H] bf16
    uint16_t* y;               // [M, H] bf16 (must not overlap x)
    const uint16_t* norm;      // [H] (1 + w) RMSNorm weight
    QMat gate, up, down;
    float eps;
    int M;
    uint64_t* hbuf;            // [kXcd][kMaxM][HWD] tagged h words
    uint64_t* pbuf;            // [kXcd][kRanks][RB][kMaxM] tagged fp32 part sums
    uint32_t* ctrl;            // [0] epoch, [16] arrivals, [32] sticky error
    int spin_limit;
};

__device__ __forceinline__ uint64_t ld_tagged(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_tagged(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool errored(const uint32_t* ctrl) {
    return __hip_atomic_load(ctrl + 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
__device__ __forceinline__ uint32_t tag_of(uint64_t w) { return (uint32_t)(w >> 32); }

constexpr int kDmaA = 2 * RA * 128 / 1024;   // gate/up DMA instructions per wave (6)
constexpr int kDmaB = 16 * (IX / 2) / 1024;  // down DMA blocks per tile (6: 16 rows x 384 bytes)
static_assert(kDmaA == 6 && kDmaB == 6, "staging shapes");

struct alignas(16) Smem {
    union {
        uint4 wgu[kWaves][kDmaA][64];            // each wave's gate/up weight lines (48 KB)
        mf::f32x4_t red[kWaves][NTA][2][64];     // gate/up wave partials, each over its wave's lines
        uint32_t hs[kMaxM][HLD];                 // the XCD's h slice, [m][k/2] bf16 pairs (48.5 KB)
    } u;
    uint4 wdn[NTB][kDmaB][64];                   // down weight lines of the four tiles (24 KB)
    uint4 nw[H / 8];                             // norm weights
    uint16_t sgu[4][RA * GA];                    // gate s, up s, gate b, up b of the 24 rows
    uint16_t sdn[2][RB * GB];                    // down s, b of the 64 rows, this part's 12 groups
    float gu[2 * RA][MP];                        // gate/up sums by weight row
    mf::f32x4_t redb[kWaves][2][64];             // down wave partials
    float part[RB][MP];                          // this workgroup's part sums
    float ss[kWaves][kMaxM];                     // per-wave sums of squares
    uint32_t epoch;
    int abort;
};

// After a failed poll round: one decision for the whole block.  Thread 0
// checks the round bound and, every 64th round, the error word (a
// device-scope round trip); on either the block gives up and sets the error
// word.  Called by every thread of the block.
__device__ __forceinline__ bool give_up(const Params& p, int tid, int spins) {
    if (__syncthreads_or(tid == 0 && (spins >= p.spin_limit || ((spins & 63) == 63 && errored(p.ctrl))))) {
        if (tid == 0) __hip_atomic_store(p.ctrl + 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    }
    __builtin_amdgcn_s_sleep(1);
    return false;
}

// Waits until each active thread's word carries `tag`: one word per producer
// (the last word it writes), polled before the producers' whole blocks are
// read, so that early rounds move a few hundred bytes instead of the blocks.
// Only a heuristic for when to read: every word read afterwards is checked
// by its own tag.  Called by every thread of the block.
__device__ __forceinline__ bool wait_sentinels(const uint64_t* word, bool active, uint32_t tag, const Params& p,
                                               int tid) {
    for (int spins = 0;; ++spins) {
        bool mine = true;
        if (active) mine = tag_of(ld_tagged(word)) == tag;
        if (__syncthreads_and(mine)) return true;
        if (give_up(p, tid, spins)) return false;
    }
}

template <int MT>
__global__ __launch_bounds__(kThreads) void mlp_rows_kernel(Params p) {
#pragma clang fp contract(off)
    __shared__ Smem sm;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c16 = lane & 15, kq = lane >> 4;
    const int wg = blockIdx.x, xj = wg % kXcd, rk = wg / kXcd;
    const int M = p.M;

    // thread 0: the epoch and the error word, ahead of the weights
    uint32_t e = 0u, err = 0u, arrived = 0u;
    if (tid == 0) {
        e = __hip_atomic_load(p.ctrl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        err = __hip_atomic_load(p.ctrl + 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- loads, in this order: norm weights, scales and biases and this
    // wave's gate/up weight lines (LDS DMA), then the activations; the down
    // weight lines follow once the sums of squares are in LDS ----
    const int g0 = wave * GWA;
    // norm weights, scales and biases by LDS DMA, lane-linear: norm 16-byte
    // chunk 64 w + lane (waves 0-3); gate/up scales and biases [gate s | up s
    // | gate b | up b] of the 24 rows, 16-byte chunk 64 w + lane (waves 0-5);
    // down scales and biases [s | b] of the 64 rows and this part's 12
    // groups, dword 128 w + 64 i + lane (waves 0-5)
    if (wave < 4)
        dma16(reinterpret_cast<const uint4*>(p.norm) + 64 * wave + lane, &sm.nw[64 * wave]);
    if (wave < 6) {
        const int c = 64 * wave + lane, a = c / 96;
        const uint16_t* src = a == 0 ? p.gate.s : a == 1 ? p.up.s : a == 2 ? p.gate.b : p.up.b;
        dma16(reinterpret_cast<const uint4*>(src + (int64_t)(xj * IX + rk * RA) * GA) + c % 96,
              reinterpret_cast<uint4*>(&sm.sgu[0][0]) + 64 * wave);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int d = 128 * wave + 64 * i + lane, a = d / 384, r = (d % 384) / 6, q = d % 6;
            const uint16_t* src = a == 0 ? p.down.s : p.down.b;
            dma4(src + (int64_t)(rk * RB + r) * (I / 64) + xj * GB + 2 * q,
                 reinterpret_cast<uint32_t*>(&sm.sdn[0][0]) + 128 * wave + 64 * i);
        }
    }
    // gate/up weight lines: the wave's 128 bytes (groups 4 w .. 4 w + 3) of
    // the 48 rows [24 gate; 24 up], block i holding rows 8 i .. 8 i + 7
#pragma unroll
    for (int i = 0; i < kDmaA; ++i) {
        const int slot = 64 * i + lane, row = slot >> 3, u = stage_chunk(slot, row);
        const uint32_t* wq = row < RA ? p.gate.wq : p.up.wq;
        const int grow = xj * IX + rk * RA + (row < RA ? row : row - RA);
        dma16(wq + (int64_t)grow * (H / 8) + 32 * wave + 4 * u, &sm.u.wgu[wave][i][0]);
    }
    // activations of the wave's groups (MFMA A layout: row m = 16 mt + c16,
    // k block kq), issued after the DMA above: loads complete in issue
    // order, so once the activations are in, so are the staged lines.  Rows
    // m >= M repeat row M - 1: an MFMA output row depends on its own A row
    // only, and those rows are never read back.
    uint4 xa[MT][GWA][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + c16;
        const int mm = m < M ? m : M - 1;
#pragma unroll
        for (int gi = 0; gi < GWA; ++gi) {
            const uint4* src = reinterpret_cast<const uint4*>(p.x + (int64_t)mm * H + 64 * (g0 + gi) + 16 * kq);
            xa[mt][gi][0] = src[0];
            xa[mt][gi][1] = src[1];
        }
    }
    // ---- sums of squares of the M rows (this wave's 256 k) ----
    // (the error word is read later; a workgroup that starts on a set error
    // word skips its work, but every workgroup computes this much first)
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
    wait_vmcnt<0>();                                   // this wave's DMA so far (read after B1)
    if (tid == 0) {
        // e sits in a register (its load has returned) before the count below
        // is issued, so no workgroup can read an epoch the count moves on
        asm volatile("" : "+v"(e) : : "memory");
        sm.epoch = e;
        sm.abort = (int)err;
        // count this workgroup in; the 256th arrival (all have read the
        // epoch) moves the epoch on for the next launch, at its end
        arrived = __hip_atomic_fetch_add(p.ctrl + 16, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // down weight lines: tile tb = wave / 2 (rows 64 r + 16 tb + [0, 16)),
    // part xj (384 bytes of each row, three lines); the tile's two waves
    // stage three blocks each and both read all six
    const int tb = wave >> 1, gb0 = GWB * (wave & 1);
#pragma unroll
    for (int i = 0; i < kDmaB / 2; ++i) {
        const int b = 3 * (wave & 1) + i;
        const int slot = 64 * b + lane, G = slot >> 3, row = G & 15, u = stage_chunk(slot, row);
        const int grow = rk * RB + 16 * tb + row;
        dma16(p.down.wq + (int64_t)grow * (I / 8) + xj * (IX / 8) + 32 * (G >> 4) + 4 * u, &sm.wdn[tb][b][0]);
    }
    // ---- barrier B1 ----
    // Barriers between phases that share only LDS carry no memory fence
    // (lds_barrier): a fence would wait for every outstanding load of the
    // wave, the weight DMA included.
    lds_barrier();                                     // B1: sums of squares, nw, sgu, sdn, epoch
    const uint32_t htag = sm.epoch * 4u + 1u, ptag = sm.epoch * 4u + 2u;
    bool ok = sm.abort == 0;
    const uint4 ones = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
    const mf::f32x4_t zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    if (ok) {
        mf::f32x4_t acc[NTA][MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            float tot = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) tot += sm.ss[w][16 * mt + c16];
            const float r = rms_inv(tot, H, p.eps);
#pragma unroll
            for (int gi = 0; gi < GWA; ++gi)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint4 v = xa[mt][gi][h], w = sm.nw[8 * (g0 + gi) + 2 * kq + h];
                    xa[mt][gi][h] = mf::pair_order(make_uint4(norm_word(v.x, w.x, r), norm_word(v.y, w.y, r),
                                                              norm_word(v.z, w.z, r), norm_word(v.w, w.w, r)));
                }
#pragma unroll
            for (int t = 0; t < NTA; ++t) acc[t][mt] = zero4;
        }
        // ---- gate/up products over the wave's 4 groups ----
#pragma unroll
        for (int gi = 0; gi < GWA; ++gi) {
            mf::f32x4_t X[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) X[mt] = mf::mfma16(xa[mt][gi][1], ones, mf::mfma16(xa[mt][gi][0], ones, zero4));
#pragma unroll
            for (int t = 0; t < NTA; ++t) {
                const int row = 16 * t + c16;
                const uint2 wv = reinterpret_cast<const uint2*>(
                    &sm.u.wgu[wave][0][0])[2 * stage_slot(row, row, 2 * gi + (kq >> 1)) + (kq & 1)];
                const uint4 b0 = mf::unpack_word(wv.x), b1 = mf::unpack_word(wv.y);
                const int sa = row < RA ? 0 : 1, sr = row < RA ? row : row - RA;
                const float s = bf16_to_f32(sm.sgu[sa][sr * GA + g0 + gi]);
                const float c = affine_c(s, sm.sgu[2 + sa][sr * GA + g0 + gi]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const mf::f32x4_t P = mf::mfma16(xa[mt][gi][1], b1, mf::mfma16(xa[mt][gi][0], b0, zero4));
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[t][mt][i] = __builtin_fmaf(s, P[i], __builtin_fmaf(c, X[mt][i], acc[t][mt][i]));
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NTA; ++t)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) sm.u.red[wave][t][mt][lane] = acc[t][mt];
    }
    lds_barrier();                                     // B3: wave partials
    // ---- wave partials in wave order -> gu[weight row][m] ----
    if (ok && tid < NTA * MT * 64) {
        const int t = tid / (MT * 64), mt = (tid / 64) % MT, l = tid & 63;
        mf::f32x4_t v = sm.u.red[0][t][mt][l];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) {
            const mf::f32x4_t o = sm.u.red[w][t][mt][l];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] += o[i];
        }
        // lane l of a tile holds rows m = 16 mt + 4 (l / 16) + i of weight row 16 t + l % 16
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.gu[16 * t + (l & 15)][16 * mt + 4 * (l >> 4) + i] = v[i];
    }
    lds_barrier();                                     // B4: gate/up sums
    // ---- SwiGLU, publish this workgroup's h words, gather the XCD's slice ----
    // (this wave's down-weight DMA has landed before the gather's first
    // barrier: the down products read both waves' blocks of their tile)
    wait_vmcnt<0>();
    uint64_t* hg = p.hbuf + (size_t)xj * kMaxM * HWD;
    if (ok && tid < M * (RA / 2)) {
        const int m = tid / (RA / 2), w = tid % (RA / 2);
        const uint32_t h0 = swiglu_bf16(sm.gu[2 * w][m], sm.gu[RA + 2 * w][m]);
        const uint32_t h1 = swiglu_bf16(sm.gu[2 * w + 1][m], sm.gu[RA + 2 * w + 1][m]);
        st_tagged(hg + (size_t)m * HWD + rk * (RA / 2) + w, ((uint64_t)htag << 32) | h0 | (h1 << 16));
    }
    {
        constexpr int PER = kMaxM * HWD / kThreads;    // 24
        const int n = M * HWD;
        __builtin_amdgcn_s_sleep(kSleep0);
        // the last word of each of the XCD's 32 producers (row M - 1, word 11
        // of its 12), then every word, re-reading only those not yet tagged
        const int ps = tid < kRanks ? tid : 0;
        if (ok) ok = wait_sentinels(hg + (size_t)(M - 1) * HWD + ps * (RA / 2) + RA / 2 - 1, tid < kRanks, htag, p, tid);
        uint64_t w[PER];
        uint32_t pend = 0u;
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (i * kThreads + tid < n) pend |= 1u << i;
        for (int spins = 0; ok; ++spins) {
#pragma unroll
            for (int i = 0; i < PER; ++i)
                if ((pend >> i) & 1u) w[i] = ld_tagged(hg + i * kThreads + tid);
#pragma unroll
            for (int i = 0; i < PER; ++i)
                if (((pend >> i) & 1u) && tag_of(w[i]) == htag) pend &= ~(1u << i);
            if (__syncthreads_and(pend == 0u)) break;
            if (give_up(p, tid, spins)) ok = false;
        }
        if (ok) {
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int k = i * kThreads + tid;
                if (k < n) sm.u.hs[k / HWD][k % HWD] = (uint32_t)w[i];
            }
        }
    }
    ok = __syncthreads_and(ok) != 0;
    // ---- down: part xj of rows rowb, the wave's 6 groups ----
    if (ok) {
        mf::f32x4_t acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = zero4;
#pragma unroll
        for (int gi = 0; gi < GWB; ++gi) {
            const int kk = 64 * (gb0 + gi) + 16 * kq;       // k within the part
            const int ch = 2 * (gb0 + gi) + (kq >> 1);          // 16-byte chunk of the part's 384-byte row
            const uint2 wv = reinterpret_cast<const uint2*>(
                &sm.wdn[tb][0][0])[2 * stage_slot(c16 + 16 * (ch >> 3), c16, ch & 7) + (kq & 1)];
            const uint4 b0 = mf::unpack_word(wv.x), b1 = mf::unpack_word(wv.y);
            const int srow = 16 * tb + c16;
            const float s = bf16_to_f32(sm.sdn[0][srow * GB + gb0 + gi]);
            const float c = affine_c(s, sm.sdn[1][srow * GB + gb0 + gi]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = 16 * mt + c16;
                const uint4* src = reinterpret_cast<const uint4*>(&sm.u.hs[m < M ? m : M - 1][kk >> 1]);
                const uint4 a0 = mf::pair_order(src[0]), a1 = mf::pair_order(src[1]);
                const mf::f32x4_t X = mf::mfma16(a1, ones, mf::mfma16(a0, ones, zero4));
                const mf::f32x4_t P = mf::mfma16(a1, b1, mf::mfma16(a0, b0, zero4));
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mt][i] = __builtin_fmaf(s, P[i], __builtin_fmaf(c, X[i], acc[mt][i]));
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) sm.redb[wave][mt][lane] = acc[mt];
    }
    lds_barrier();                                     // B5: down wave partials
    // ---- the two waves of each tile, in order -> part[row][m] ----
    if (ok && tid < NTB * MT * 64) {
        const int t = tid / (MT * 64), mt = (tid / 64) % MT, l = tid & 63;
        const mf::f32x4_t a = sm.redb[2 * t][mt][l], b = sm.redb[2 * t + 1][mt][l];
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.part[16 * t + (l & 15)][16 * mt + 4 * (l >> 4) + i] = a[i] + b[i];
    }
    lds_barrier();                                     // B6: part sums
    // ---- publish the part sums; gather this workgroup's 8 rows from every XCD ----
    uint64_t* pw = p.pbuf + ((size_t)xj * kRanks + rk) * RB * kMaxM;
    if (ok) {
        for (int k = tid; k < RB * M; k += kThreads) {
            const int row = k / M, m = k % M;
            st_tagged(pw + (size_t)row * kMaxM + m, ((uint64_t)ptag << 32) | __float_as_uint(sm.part[row][m]));
        }
    }
    const int oi = tid / kMaxM, om = tid % kMaxM;      // (row, m) of this thread's output
    const bool owner = tid < ROUT * kMaxM && om < M;
    const int orow = rk * RB + ROUT * xj + oi;          // global hidden row
    uint64_t pw8[kXcd];
    {
        __builtin_amdgcn_s_sleep(kSleep0);
        // the last word of each of the 8 producers of this row block (row 63,
        // m = M - 1), then this thread's 8 words, re-reading untagged ones
        const int js = tid < kXcd ? tid : 0;
        if (ok)
            ok = wait_sentinels(p.pbuf + (((size_t)js * kRanks + rk) * RB + RB - 1) * kMaxM + M - 1, tid < kXcd, ptag,
                                p, tid);
        uint32_t pend = owner ? (1u << kXcd) - 1u : 0u;
        for (int spins = 0; ok; ++spins) {
#pragma unroll
            for (int j = 0; j < kXcd; ++j)
                if ((pend >> j) & 1u)
                    pw8[j] = ld_tagged(p.pbuf + (((size_t)j * kRanks + rk) * RB + ROUT * xj + oi) * kMaxM + om);
#pragma unroll
            for (int j = 0; j < kXcd; ++j)
                if (((pend >> j) & 1u) && tag_of(pw8[j]) == ptag) pend &= ~(1u << j);
            if (__syncthreads_and(pend == 0u)) break;
            if (give_up(p, tid, spins)) ok = false;
        }
    }
    ok = __syncthreads_and(ok) != 0;
    if (owner) {
        const int64_t o = (int64_t)om * H + orow;
        if (ok) {
            float yv = __uint_as_float((uint32_t)pw8[0]);
#pragma unroll
            for (int j = 1; j < kXcd; ++j) yv += __uint_as_float((uint32_t)pw8[j]);
            p.y[o] = (uint16_t)f32_to_bf16(bf16_to_f32(p.x[o]) + round_bf16(yv));
        } else {
            p.y[o] = 0x7fc0u;                           // NaN: the launch timed out
        }
    }
    asm volatile("" : "+v"(arrived));                  // its atomic is waited for here, not earlier
    if (tid == 0 && arrived % kNWG == kNWG - 1)
        __hip_atomic_store(p.ctrl, e + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace rows

// Co-residency of the 256 workgroups, checked once per device.
constexpr int kMaxRowsDevices = 64;
static int g_rows_ok[kMaxRowsDevices][2];
static bool g_rows_checked[kMaxRowsDevices][2];
static std::mutex g_rows_mu;
constexpr int kRowsSpinLimit = 1 << 20;

}  // namespace mq4

using namespace mq4;

extern "C" size_t mq4_mlp_layers_workspace_size(int64_t M, int64_t hidden, int64_t intermediate) {
    if (M < 1 || M > rows::kMaxM || hidden != rows::H || intermediate != rows::I) return 0;
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    // ctrl + h words + part sums + two ping-pong hidden states for stacks of layers
    return 256 + up((size_t)rows::kXcd * rows::kMaxM * rows::HWD * 8) +
           up((size_t)rows::kXcd * rows::kRanks * rows::RB * rows::kMaxM * 8) + 2 * up((size_t)M * hidden * 2);
}

extern "C" int mq4_mlp_layers(const uint16_t* x_in, int64_t M, int64_t hidden, int64_t intermediate,
                              int64_t n_layers, const mq4_mlp_layer* layers, float eps, uint16_t* x_out,
                              void* workspace, size_t workspace_bytes, void* stream) {
    const char* what = "mq4_mlp_layers";
    if (hidden != rows::H || intermediate != rows::I)
        return fail(MQ4_ERR_UNSUPPORTED, "%s: built for hidden=%d, intermediate=%d (got %lld, %lld)", what, rows::H,
                    rows::I, (long long)hidden, (long long)intermediate);
    if (M < 1 || M > rows::kMaxM)
        return fail(MQ4_ERR_UNSUPPORTED, "%s: M must be in [1, %d] (got %lld)", what, rows::kMaxM, (long long)M);
    if (n_layers < 1 || n_layers > 1024) return fail(MQ4_ERR_INVALID_ARG, "%s: n_layers must be in [1, 1024]", what);
    if (!x_in || !x_out || !layers) return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    if (!aligned(x_in, 16) || !aligned(x_out, 16))
        return fail(MQ4_ERR_ALIGNMENT, "%s: x_in and x_out must be 16-byte aligned", what);
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(x_in), a1 = reinterpret_cast<uintptr_t>(x_out);
    const uintptr_t nb = (uintptr_t)M * hidden * 2;
    if (a0 < a1 + nb && a1 < a0 + nb)
        return fail(MQ4_ERR_INVALID_ARG, "%s: x_out must not overlap x_in", what);
    const size_t need = mq4_mlp_layers_workspace_size(M, hidden, intermediate);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
        return fail(MQ4_ERR_WORKSPACE, "%s: workspace needs %zu bytes, 256-byte aligned, zero-filled once", what,
                    need);
    const uintptr_t w0 = reinterpret_cast<uintptr_t>(workspace);
    if ((a0 < w0 + need && w0 < a0 + nb) || (a1 < w0 + need && w0 < a1 + nb))
        return fail(MQ4_ERR_INVALID_ARG, "%s: x_in and x_out must not overlap the workspace", what);
    for (int64_t l = 0; l < n_layers; ++l) {
        const mq4_mlp_layer& s = layers[l];
        if (!s.norm_weight || !s.gate_wq || !s.gate_scales || !s.gate_biases || !s.up_wq || !s.up_scales ||
            !s.up_biases || !s.down_wq || !s.down_scales || !s.down_biases)
            return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer in layer %lld", what, (long long)l);
        if (!aligned(s.norm_weight, 16) || !aligned(s.gate_wq, 16) || !aligned(s.up_wq, 16) ||
            !aligned(s.down_wq, 16) || !aligned(s.gate_scales, 16) || !aligned(s.gate_biases, 16) ||
            !aligned(s.up_scales, 16) || !aligned(s.up_biases, 16) || !aligned(s.down_scales, 16) ||
            !aligned(s.down_biases, 16))
            return fail(MQ4_ERR_ALIGNMENT, "%s: layer %lld norm weight, packed weights, scales and biases must be "
                        "16-byte aligned", what, (long long)l);
    }
    const int mt = M > 16 ? 1 : 0;
    const void* kern = mt ? reinterpret_cast<const void*>(rows::mlp_rows_kernel<2>)
                          : reinterpret_cast<const void*>(rows::mlp_rows_kernel<1>);
    {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxRowsDevices)
            return fail(MQ4_ERR_HIP, "%s: hipGetDevice failed", what);
        std::lock_guard<std::mutex> lk(g_rows_mu);
        if (!g_rows_checked[dev][mt]) {
            int cus = 0, occ = 0;
            if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, rows::kThreads, 0) != hipSuccess)
                return fail(MQ4_ERR_HIP, "%s: device query failed", what);
            g_rows_ok[dev][mt] = (cus >= rows::kNWG && occ >= 1) ? 1 : 0;
            g_rows_checked[dev][mt] = true;
        }
        if (g_rows_ok[dev][mt] == 0)
            return fail(MQ4_ERR_UNSUPPORTED, "%s: needs %d co-resident workgroups of %d threads", what, rows::kNWG,
                        rows::kThreads);
    }
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    char* ws = reinterpret_cast<char*>(workspace);
    const size_t hw = up((size_t)rows::kXcd * rows::kMaxM * rows::HWD * 8),
                 pw = up((size_t)rows::kXcd * rows::kRanks * rows::RB * rows::kMaxM * 8), xw = up((size_t)nb);
    rows::Params p{};
    p.ctrl = reinterpret_cast<uint32_t*>(ws);
    p.hbuf = reinterpret_cast<uint64_t*>(ws + 256);
    p.pbuf = reinterpret_cast<uint64_t*>(ws + 256 + hw);
    uint16_t* ping[2] = {reinterpret_cast<uint16_t*>(ws + 256 + hw + pw),
                         reinterpret_cast<uint16_t*>(ws + 256 + hw + pw + xw)};
    p.M = (int)M;
    p.eps = eps;
    p.spin_limit = kRowsSpinLimit;
    hipStream_t st = as_stream(stream);
    for (int64_t l = 0; l < n_layers; ++l) {
        const mq4_mlp_layer& s = layers[l];
        p.x = l == 0 ? x_in : ping[(l - 1) & 1];
        p.y = l == n_layers - 1 ? x_out : ping[l & 1];
        p.norm = s.norm_weight;
        p.gate = {s.gate_wq, s.gate_scales, s.gate_biases};
        p.up = {s.up_wq, s.up_scales, s.up_biases};
        p.down = {s.down_wq, s.down_scales, s.down_biases};
        if (mt)
            hipLaunchKernelGGL(rows::mlp_rows_kernel<2>, dim3(rows::kNWG), dim3(rows::kThreads), 0, st, p);
        else
            hipLaunchKernelGGL(rows::mlp_rows_kernel<1>, dim3(rows::kNWG), dim3(rows::kThreads), 0, st, p);
    }
    return launch_status(what);
}
