// Persistent single-launch decode step (M = 1) for gfx950:
//
//   for each layer l:  n = rms_norm(x, norm_l);  h = swiglu(n @ Wg^T, n @ Wu^T)
//                      x = x + h @ Wd^T
//   token = argmax(rms_norm(x, final_norm) @ Wlm^T)
//
// i.e. the per-token loop of src/model/marlin.cpp:110-145 restricted to the
// MLP half of each layer (rms_norm :141, mlp_forward :31-35, residual :142),
// then the final norm (:145), lm_head (:161-169) and greedy sample_token
// (src/sampling/sampler.cpp:14-16), with the same arithmetic as the separate
// kernels of mq4_gemv.hip.  With vocab = 0 the launch ends after the layers
// (one MLP half per call, as the reference's layer loop needs between its
// attention / SSM halves).
//
// Why one launch: the step is 2 * layers + 1 dependent phases.  Separate
// kernels drain the memory pipeline at every boundary (every phase pays the
// full HBM latency); here the weights, which never depend on activations,
// are loaded one phase ahead into the compute waves' registers, so the HBM
// stream keeps running while the small activation vectors are exchanged.
//
// Exchange without fences or read-modify-write atomics: both measured slow
// on MI355X (a device-scope release fence writes back the L2; RMW atomics to
// one address serialize).  Activations travel as 64-bit words, two bf16
// values in the low half and a 32-bit phase tag in the high half, written
// and read with relaxed device-scope atomic stores/loads.  A consumer polls
// the words it needs until every tag equals the phase's tag; each word is
// self-validating (single-location coherence), so no ordering between
// different words is needed.  Buffers are rewritten every layer and a phase
// only overwrites words whose previous contents every consumer has already
// read (a workgroup can only reach the next write after all workgroups
// produced the inputs that depended on the previous read).
//
// Workgroup roles: 4 I/O waves poll and publish activations and stage them
// in LDS (pre-paired for the dot2 layout); 8 compute waves hold weights in
// registers and only touch LDS, so their loads stay in flight across the
// workgroup barriers (on gfx950 a barrier waits for LDS only, not for
// outstanding global loads).  Every wait is bounded: on a timeout a sticky
// error word is set, every workgroup leaves, and the token reads 0xFFFFFFFF.
#include <mutex>

#include "mq4_device.h"
#include "mq4_host.h"
#include "mq4_stage.h"

namespace mq4 {

namespace dec {

constexpr int kNWG = 256;            // workgroups (one per CU)
constexpr int kNIO = 4;              // I/O waves per workgroup
constexpr int kNCW = 8;              // compute waves per workgroup
constexpr int kThreads = 64 * (kNIO + kNCW);
constexpr int kMaxLayers = 32;
constexpr int kCopies = 8;           // replicas of the exchange buffers (one per XCD)
constexpr int kFirstPollSleep = 28;  // s_sleep units (64 clocks) before the first poll round
constexpr int H = 2048;              // hidden size this instance is built for
constexpr int I = 6144;              // intermediate size
constexpr int SA = H / 32;           // 16-byte slices per gate/up row (64)
constexpr int SB = I / 32;           // slices per down row (192)
constexpr int SPL_B = SB / 64;       // down slices per lane (3)
constexpr int RA = I / kNWG / kNCW;  // gate/up rows per compute wave (3)
constexpr int RB = H / kNWG / kNCW;  // down rows per compute wave (1)
constexpr int LM_RPI = 4;            // lm_head rows per batch
constexpr int LM_NBUF = 3;           // lm_head batches in flight per compute wave
static_assert(SA == 64 && SB % 64 == 0 && RA * kNWG * kNCW == I && RB * kNWG * kNCW == H, "shape");

struct Layer {
    const uint16_t* norm;
    QMat gate, up, down;
};

struct Params {
    const uint16_t* x_in;      // [H] bf16
    uint16_t* x_out;           // [H] bf16 hidden state after the last layer (may be null)
    uint32_t* idx;             // [1] token (unused when vocab == 0)
    const uint16_t* final_norm;
    float eps;
    QMat lm;
    int vocab;                 // 0: layers only (no final norm, lm_head or token)
    int n_layers;
    uint64_t* xbuf;            // [kCopies][H/2] tagged words
    uint64_t* hbuf;            // [kCopies][I/2] tagged words
    uint64_t* part;            // [kNWG] tagged per-workgroup argmax keys
    uint32_t* ctrl;            // [0] epoch, [32] sticky error flag
    int spin_limit;
    Layer layers[kMaxLayers];
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
__device__ __forceinline__ void set_error(uint32_t* ctrl) {
    __hip_atomic_store(ctrl + 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Poll NW tagged words starting at src (NW a multiple of 64) until every tag
// equals `tag`; store the 2*NW bf16 values to dst.  false on timeout/abort.
// One round in flight: a second, staggered round doubles the poll traffic,
// and all polls slow down by more than the finer sampling gains.  (Packing
// three bf16 and a 16-bit tag per word measured slower too: the scattered
// 16-bit LDS unpack costs more than the saved poll bytes.)
template <int NW>
__device__ bool poll_words(const uint64_t* src, uint32_t tag, uint32_t* dst, const Params& p, int lane) {
    constexpr int PER = NW / 64;
    uint64_t w[PER];
    // The first round is delayed by 28 x 64 clocks (~0.75 us): issued right
    // after this workgroup's own publish it meets the other workgroups'
    // stores still in flight and takes ~1.5 us to return (and fails), while a
    // round issued later returns in ~0.6 us with the phase complete.  (Swept
    // on MI355X: 12-48 units give 207-212 us per step at the ends, 195 us at
    // 24-32; separate delays for the x and h exchanges gain nothing.)
    __builtin_amdgcn_s_sleep(kFirstPollSleep);
    for (int spins = 0;; ++spins) {
#pragma unroll
        for (int i = 0; i < PER; ++i) w[i] = ld_tagged(src + i * 64 + lane);
        bool ok = true;
#pragma unroll
        for (int i = 0; i < PER; ++i) ok &= (uint32_t)(w[i] >> 32) == tag;
        if (__all(ok)) break;
        if (spins >= p.spin_limit || errored(p.ctrl)) {
            if (lane == 0) set_error(p.ctrl);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) dst[i * 64 + lane] = (uint32_t)w[i];
    return true;
}

// Per-compute-wave LDS staging of one layer's weights (filled by LDS DMA):
// gate/up rows rowA..rowA+RA-1 of both matrices, and the down row.
struct alignas(16) WStageA {
    uint4 w[2][RA][64];            // 16-byte slices, lane-major
    uint32_t s[2][64];             // the RA*32 bf16 scales of each matrix (dwords 0..47)
    uint32_t b[2][64];             // biases, same layout
};
struct alignas(16) WStageB {
    uint4 w[SPL_B][64];
    uint32_t s[64];                // the 96 bf16 scales of the down row (dwords 0..47)
    uint32_t b[64];
};
constexpr int kDmaA = 2 * (RA + 2);  // LDS DMA instructions per gate/up stage
constexpr int kDmaB = SPL_B + 2;     // per down stage


// Pin a value in a VGPR at this point of the program: the computation that
// produces it cannot be moved below (e.g. below a barrier) by the compiler.
__device__ __forceinline__ void pin(uint32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }


struct alignas(16) Smem {
    uint32_t xraw[H / 2];          // raw x of the current layer (residual), bf16 pairs
    uint4 xp[4][SA];               // dot2-paired normalized x: chunk w of slice s at [w][s]
    float xs[SA];
    uint32_t hraw[I / 2];          // h as polled
    uint4 hp[4][SB];               // dot2-paired h, same chunk-major layout (conflict-free reads)
    float hs[SB];
    uint32_t out[32];              // this workgroup's outputs (bf16 in the low half)
    uint64_t best[kNCW];
    uint32_t epoch;
    int abort;
};

// dot2 part of one slice: D = sum_k x_k*(128 + q_k) over its 32 elements.
__device__ __forceinline__ float slice_d(const uint4& w, const uint32_t* xp) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    float d = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        d = dot2_bf16(xp[4 * k + 0], nib_pair_bf16<0>(wd[k]), d);
        d = dot2_bf16(xp[4 * k + 1], nib_pair_bf16<1>(wd[k]), d);
        d = dot2_bf16(xp[4 * k + 2], nib_pair_bf16<2>(wd[k]), d);
        d = dot2_bf16(xp[4 * k + 3], nib_pair_bf16<3>(wd[k]), d);
    }
    return d;
}

// The same dot2 chain over pre-unpacked nibble pairs (nib_pairs of the four words).
__device__ __forceinline__ float pairs_d(const uint32_t* pr, const uint32_t* xp) {
    float d = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) d = dot2_bf16(xp[i], pr[i], d);
    return d;
}

// (1 + w) RMSNorm of x into xp/xs.  Every I/O wave computes the full sum of
// squares (lane l sums the 16 words of slice l, then the wave reduces: the
// order of the separate kernels) and handles a quarter of the slices, 4 lanes
// per slice, one 16-byte chunk per lane (chunk io*64 + lane of x); nw is this
// lane's chunk of the norm weight, loaded a layer ahead.
__device__ __forceinline__ float norm_rinv(const uint4 (&v)[4], float eps) {
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        ss = sumsq_word(ss, v[k].x);
        ss = sumsq_word(ss, v[k].y);
        ss = sumsq_word(ss, v[k].z);
        ss = sumsq_word(ss, v[k].w);
    }
    ss = wave_sum(ss);
    return rms_inv(ss, H, eps);
}
__device__ __forceinline__ void norm_chunk(Smem& sm, const uint4 nw, float r, const uint4 xv, int io, int lane) {
    constexpr int SPW = SA / kNIO;                 // 16 slices per I/O wave
    const int sl = io * SPW + (lane >> 2);
    const int q = lane & 3;
    const uint4 xn = make_uint4(norm_word(xv.x, nw.x, r), norm_word(xv.y, nw.y, r), norm_word(xv.z, nw.z, r),
                                norm_word(xv.w, nw.w, r));
    uint32_t pr[4];
    const float c = pair_chunk(xn, pr, 0.0f);
    sm.xp[q][sl] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
    const float c1 = quad_lane<1>(c), c2 = quad_lane<2>(c), c3 = quad_lane<3>(c);
    if (q == 0) sm.xs[sl] = ((c + c1) + c2) + c3;
}
// The same from x in xraw (all I/O waves' quarters, after a barrier).
__device__ void stage_norm_x(Smem& sm, const uint4 nw, float eps, int io, int lane) {
    const uint4* x4 = reinterpret_cast<const uint4*>(sm.xraw);
    const uint4 v[4] = {x4[lane * 4], x4[lane * 4 + 1], x4[lane * 4 + 2], x4[lane * 4 + 3]};
    norm_chunk(sm, nw, norm_rinv(v, eps), x4[io * 64 + lane], io, lane);
}

// Pair the polled h (this wave's quarter of the slices): 4 lanes per slice,
// one 16-byte chunk each.  The slice sum ((c0 + c1) + c2) + c3 of the chunk
// sums c = 0 + C equals the separate kernels' (((0 + C0) + C1) + C2) + C3 (no
// partial sum can be -0, so the extra + 0 never changes a bit).
__device__ void stage_h(Smem& sm, int io, int lane) {
    constexpr int SPW = SB / kNIO;    // 48 slices per wave, 16 per pass
    const int q = lane & 3;
#pragma unroll
    for (int pass = 0; pass < SPW / 16; ++pass) {
        const int sl = io * SPW + pass * 16 + (lane >> 2);
        uint32_t pr[4];
        const float c = pair_chunk(reinterpret_cast<const uint4*>(sm.hraw)[sl * 4 + q], pr, 0.0f);
        sm.hp[q][sl] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
        const float c1 = quad_lane<1>(c), c2 = quad_lane<2>(c), c3 = quad_lane<3>(c);
        if (q == 0) sm.hs[sl] = ((c + c1) + c2) + c3;
    }
}

__global__ __launch_bounds__(kThreads) void decode_step_kernel(Params p) {
    __shared__ Smem sm;
    __shared__ WStageA wsa[kNCW];
    __shared__ WStageB wsb[kNCW];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wg = blockIdx.x;
    const int L = p.n_layers;

    // LDS DMA of one layer's weights into compute wave c's staging buffers.
    const int sdw = lane < 48 ? lane : 47;           // dword of a 192-byte scale/bias run
    auto dmaA = [&](int c, int l, int t) {           // kDmaA / 2 instructions (t: 0 gate, 1 up)
        const Layer& Ly = p.layers[l];
        const int rowA = wg * (I / kNWG) + c * RA;
        {
            const QMat& Q = t == 0 ? Ly.gate : Ly.up;
#pragma unroll
            for (int r = 0; r < RA; ++r)
                __builtin_amdgcn_global_load_lds(
                    reinterpret_cast<const uint4*>(Q.wq + (int64_t)(rowA + r) * (H / 8)) + lane, &wsa[c].w[t][r][0], 16, 0,
                    0);
            // scales/biases of the RA consecutive rows: RA*32 bf16 = 192 bytes
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(Q.s + (int64_t)rowA * (H / 64)) + sdw,
                                             &wsa[c].s[t][0], 4, 0, 0);
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(Q.b + (int64_t)rowA * (H / 64)) + sdw,
                                             &wsa[c].b[t][0], 4, 0, 0);
        }
    };
    auto dmaB = [&](int c, int l) {                  // kDmaB instructions
        const QMat& Q = p.layers[l].down;
        const int rowB = wg * (H / kNWG) + c * RB;
#pragma unroll
        for (int j = 0; j < SPL_B; ++j)
            __builtin_amdgcn_global_load_lds(
                reinterpret_cast<const uint4*>(Q.wq + (int64_t)rowB * (I / 8)) + j * 64 + lane, &wsb[c].w[j][0], 16, 0, 0);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(Q.s + (int64_t)rowB * (I / 64)) + sdw,
                                         &wsb[c].s[0], 4, 0, 0);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(Q.b + (int64_t)rowB * (I / 64)) + sdw,
                                         &wsb[c].b[0], 4, 0, 0);
    };
    // The same for layer 0 at the start of the launch, issued as inline
    // assembly that the compiler does not track (it would otherwise wait for
    // every outstanding DMA of the wave before its next LDS read); the
    // issuing wave waits for them itself by exact counts.
    auto dmaA0 = [&](int c, int t) {                 // kDmaA / 2 instructions
        const QMat& Q = t == 0 ? p.layers[0].gate : p.layers[0].up;
        const int rowA = wg * (I / kNWG) + c * RA;
#pragma unroll
        for (int r = 0; r < RA; ++r)
            stage::dma16(reinterpret_cast<const uint4*>(Q.wq + (int64_t)(rowA + r) * (H / 8)) + lane,
                         &wsa[c].w[t][r][0]);
        stage::dma4(reinterpret_cast<const uint32_t*>(Q.s + (int64_t)rowA * (H / 64)) + sdw, &wsa[c].s[t][0]);
        stage::dma4(reinterpret_cast<const uint32_t*>(Q.b + (int64_t)rowA * (H / 64)) + sdw, &wsa[c].b[t][0]);
    };
    auto dmaB0 = [&](int c) {                        // kDmaB instructions
        const QMat& D = p.layers[0].down;
        const int rowB = wg * (H / kNWG) + c * RB;
#pragma unroll
        for (int j = 0; j < SPL_B; ++j)
            stage::dma16(reinterpret_cast<const uint4*>(D.wq + (int64_t)rowB * (I / 8)) + j * 64 + lane, &wsb[c].w[j][0]);
        stage::dma4(reinterpret_cast<const uint32_t*>(D.s + (int64_t)rowB * (I / 64)) + sdw, &wsb[c].s[0]);
        stage::dma4(reinterpret_cast<const uint32_t*>(D.b + (int64_t)rowB * (I / 64)) + sdw, &wsb[c].b[0]);
    };
    static_assert(kNCW == 2 * kNIO, "each I/O wave stages the weights of two compute waves");
    static_assert(kDmaA % 2 == 0, "gate and up halves");

    // Layer 0 starts as early as the launch allows.  The I/O waves load x and
    // the first norm weight before any weight DMA is issued in this CU (a
    // CU's loads return in issue order: one issued behind a layer's 83 KB of
    // weights waits for all of them), and thread 0 reads the epoch and the
    // error word meanwhile.  Right after B0 each compute wave DMAs its
    // layer-0 gate and up rows (issue is paced by HBM: about 2 us for a CU's
    // 55 KB), and unpacks the gate rows as soon as they land; the I/O waves
    // normalize x and then DMA the down rows.  The epoch and the error word
    // are first read after B1 (an aborted launch leaves there), so the
    // weight stream starts before the epoch is known.  (The two roles branch
    // apart before their first loads, so that the compiler's waits for the
    // I/O waves' loads do not reach the compute waves' code.)
    const int io = wave;                             // I/O wave index (wave < kNIO)
    // this lane's 16-byte chunk of a norm weight (slice io*16 + lane/4,
    // chunk lane%4), loaded one layer ahead of its use
    const int nchunk = (io * (SA / kNIO) + (lane >> 2)) * 4 + (lane & 3);
    auto norm_of = [&](int l) { return l < L ? p.layers[l].norm : p.final_norm; };
    if (wave < kNIO) {
        // ============================ I/O waves ============================
        uint4 nw = reinterpret_cast<const uint4*>(norm_of(0))[nchunk];    // L > 0 or vocab > 0
        const uint4* x4 = reinterpret_cast<const uint4*>(p.x_in);
        const uint4 xv = x4[io * 64 + lane];        // chunk io*64 + lane of x
        uint4 xa[4];                                 // slice `lane` of x (16 words)
#pragma unroll
        for (int k = 0; k < 4; ++k) xa[k] = x4[lane * 4 + k];
        // (read by every lane: a load in a one-lane branch is awaited at the
        // branch's end, which would hold B0 until the loads above return)
        const uint32_t epoch0 = __hip_atomic_load(p.ctrl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t err0 = __hip_atomic_load(p.ctrl + 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lds_barrier();                               // B0: x, norm and epoch loads issued
        if (threadIdx.x == 0) {                      // read by every wave after B1
            sm.epoch = epoch0;
            sm.abort = err0 != 0u ? 1 : 0;
        }
        uint32_t base = 0;  // phase tags base + [0, 2*layers+1]: never 0, disjoint per call (set after B1)
        // Weights reach the compute waves' LDS staging buffers by DMA, issued
        // only in phases without a poll in flight (weight traffic ahead of a
        // poll in the CU's memory pipeline delays it) and by waves idle in
        // that phase, since issuing stalls the issuing wave for about the
        // transfer time (~0.9 us for 28 KB per CU at its HBM share):
        //   gate rows of layer l+1: each compute wave, RMSNorm phase of l;
        //   up rows of layer l+1:   I/O waves, gate/up phase of l, waited by B5;
        //   down row of layer l+1:  I/O waves, down phase of l, waited by B3 of l+1.
        // Layer 0: see above.
        // I/O wave io serves compute waves 2*io and 2*io+1.  The barriers
        // carry no memory fence (lds_barrier): a fence would wait for all
        // outstanding DMA.
        // the copy of the exchange buffers this workgroup reads
        const uint64_t* xcopy = p.xbuf + (size_t)(wg % kCopies) * (H / 2);
        const uint64_t* hcopy = p.hbuf + (size_t)(wg % kCopies) * (I / 2);
        constexpr int kIoA = kDmaA, kIoB = 2 * kDmaB;   // up halves of two waves; two down rows
        // layer 0: x into xraw (the residual) and its RMSNorm straight from
        // the registers, while the weights are still streaming in
        *reinterpret_cast<uint4*>(&sm.xraw[io * (H / 2 / kNIO) + lane * 4]) = xv;
        if (L == 0 && wg == 0 && p.x_out) {
            uint32_t* xo = reinterpret_cast<uint32_t*>(p.x_out) + io * (H / 2 / kNIO) + lane * 4;
            xo[0] = xv.x, xo[1] = xv.y, xo[2] = xv.z, xo[3] = xv.w;
        }
        norm_chunk(sm, nw, norm_rinv(xa, p.eps), xv, io, lane);
        if (L > 0) {                                 // layer 0's down rows, waited before B3
            dmaB0(2 * io);
            dmaB0(2 * io + 1);
        }
        for (int l = 0; l <= L; ++l) {
            // layers only: the last layer's x_out is written; nothing reads
            // x words in this launch after it
            if (l == L && p.vocab == 0) break;
            // ---- x of layer l > 0 -> xraw (layer 0's was stored above) ----
            if (l > 0 && !poll_words<H / 2 / kNIO>(xcopy + io * (H / 2 / kNIO), base + 2 * l,
                                                   sm.xraw + io * (H / 2 / kNIO), p, lane)) {
                sm.abort = 1;
            }
            lds_barrier();                                     // B1: xraw complete
            if (sm.abort) break;
            if (l == 0) base = sm.epoch * 128u + 1u;
            if (l > 0) stage_norm_x(sm, nw, p.eps, io, lane);
            lds_barrier();                                     // B2: xp/xs ready
            if (l == L) break;
            if (l + 1 < L || p.vocab > 0) nw = reinterpret_cast<const uint4*>(norm_of(l + 1))[nchunk];
            if (l + 1 < L) {
                dmaA(2 * io, l + 1, 1);
                dmaA(2 * io + 1, l + 1, 1);
                wait_vmcnt<kIoA>();                            // down weights of layer l staged
            } else {
                wait_vmcnt<0>();
            }
            lds_barrier();                                     // B3: h slice in sm.out
            {   // this workgroup's h words into every copy
                constexpr int HW = I / kNWG / 2;
                const int i = io * 64 + lane;
                if (i < HW * kCopies) {
                    const int c = i / HW, w = i - c * HW;
                    st_tagged(p.hbuf + (size_t)c * (I / 2) + wg * HW + w,
                              ((uint64_t)(base + 2 * l + 1) << 32) | (sm.out[2 * w] | (sm.out[2 * w + 1] << 16)));
                }
            }
            if (!poll_words<I / 2 / kNIO>(hcopy + io * (I / 2 / kNIO), base + 2 * l + 1,
                                          sm.hraw + io * (I / 2 / kNIO), p, lane))
                sm.abort = 1;
            // the words this wave polled are exactly the slices it pairs
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            stage_h(sm, io, lane);
            lds_barrier();                                     // B4: hp/hs ready
            if (sm.abort) break;
            if (p.vocab == 0 && l == L - 1 && wg == 0 && io == 0 && lane == 0) {
                // layers only (no final gather): the last layer's h words came
                // from every workgroup, so every one has read the epoch; the
                // next call may take the next one
                __hip_atomic_store(p.ctrl, sm.epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (l + 1 < L) {
                dmaB(2 * io, l + 1);
                dmaB(2 * io + 1, l + 1);
                wait_vmcnt<kIoB>();                            // up weights of layer l+1 staged
            }
            lds_barrier();                                     // B5: new x rows in sm.out
            {   // this workgroup's new x words into every copy (layers only:
                // not after the last layer, whose words nothing reads)
                constexpr int XW = H / kNWG / 2;
                const int i = io * 64 + lane;
                if (i < XW * kCopies) {
                    const int c = i / XW, w = i - c * XW;
                    const uint32_t v = sm.out[2 * w] | (sm.out[2 * w + 1] << 16);
                    if (p.vocab > 0 || l + 1 < L)
                        st_tagged(p.xbuf + (size_t)c * (H / 2) + wg * XW + w,
                                  ((uint64_t)(base + 2 * l + 2) << 32) | v);
                    if (c == 0 && l == L - 1 && p.x_out) reinterpret_cast<uint32_t*>(p.x_out)[wg * XW + w] = v;
                }
            }
        }
        wait_vmcnt<0>();                                       // no DMA may outlive the workgroup
        // ---- argmax: this workgroup's best key, then workgroup 0 reduces ----
        __syncthreads();                                       // B6: sm.best filled
        if (p.vocab == 0) return;
        const uint32_t tag16 = (sm.epoch % 65535u) + 1u;
        if (!sm.abort && io == 0) {
            uint64_t b = lane < kNCW ? sm.best[lane] : 0ull;
            b = wave_max_u64(b);
            if (lane == 0) st_tagged(p.part + wg, ((uint64_t)tag16 << 48) | (b & 0xffffffffffffull));
            if (wg == 0) {
                uint64_t w[kNWG / 64];
                bool ok = false;
                for (int spins = 0;; ++spins) {
#pragma unroll
                    for (int i = 0; i < kNWG / 64; ++i) w[i] = ld_tagged(p.part + i * 64 + lane);
                    bool good = true;
#pragma unroll
                    for (int i = 0; i < kNWG / 64; ++i) good &= (uint32_t)(w[i] >> 48) == tag16;
                    if (__all(good)) { ok = true; break; }
                    if (spins >= p.spin_limit || errored(p.ctrl)) { if (lane == 0) set_error(p.ctrl); break; }
                    __builtin_amdgcn_s_sleep(1);
                }
                uint64_t bb = 0;
#pragma unroll
                for (int i = 0; i < kNWG / 64; ++i) {
                    const uint64_t k = w[i] & 0xffffffffffffull;
                    bb = k > bb ? k : bb;
                }
                bb = wave_max_u64(bb);
                if (lane == 0) {
                    p.idx[0] = ok ? argmax_key_index(bb) : 0xffffffffu;
                    if (ok) __hip_atomic_store(p.ctrl, sm.epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        } else if (sm.abort && wg == 0 && io == 0 && lane == 0) {
            p.idx[0] = 0xffffffffu;
        }
        return;
    }

    // ============================ compute waves ============================
    const int cw = wave - kNIO;
    lds_barrier();                                   // B0
    if (L > 0) {
        dmaA0(cw, 0);
        dmaA0(cw, 1);
    }
    // This wave's weights arrive in its LDS staging buffers by DMA (no
    // registers held while in flight): its gate rows by its own DMA (layer 0:
    // gate and up rows, issued right after B0), the other rows by the I/O
    // waves.  They are unpacked into bf16 nibble pairs while the activations
    // are being exchanged: gate/up weights of layer l after B5 of layer l-1,
    // down weights after B3.  The compute waves' only memory operations are
    // their own DMAs, awaited by vmcnt, so their barriers carry no fence
    // (lds_barrier).
    WStageA& SA_ = wsa[cw];
    WStageB& SB_ = wsb[cw];
    const int rowB = wg * (H / kNWG) + cw * RB;     // down row of this wave
    static_assert(RB == 1 && SPL_B == 3, "down layout");

    uint32_t pa[2][RA][16];
    float ks_a[2][RA], kc_a[2][RA];
    auto unpackA = [&](int t) {                      // t: 0 gate, 1 up
#pragma unroll
        for (int r = 0; r < RA; ++r) {
            const uint4 w = SA_.w[t][r][lane];
            nib_pairs(w.x, &pa[t][r][0]);
            nib_pairs(w.y, &pa[t][r][4]);
            nib_pairs(w.z, &pa[t][r][8]);
            nib_pairs(w.w, &pa[t][r][12]);
            const int g = r * (H / 64) + (lane >> 1);
            ks_a[t][r] = bf16_to_f32(reinterpret_cast<const uint16_t*>(SA_.s[t])[g]);
            kc_a[t][r] = affine_c(ks_a[t][r], reinterpret_cast<const uint16_t*>(SA_.b[t])[g]);
        }
        // done now, while the exchange runs, not after the next barrier
#pragma unroll
        for (int r = 0; r < RA; ++r) {
#pragma unroll
            for (int i = 0; i < 16; ++i) pin(pa[t][r][i]);
            pin(ks_a[t][r]);
            pin(kc_a[t][r]);
        }
    };
    uint32_t pb[SPL_B][16];
    float ks_b[SPL_B], kc_b[SPL_B];
    auto unpackB = [&]() {
#pragma unroll
        for (int j = 0; j < SPL_B; ++j) {
            const uint4 w = SB_.w[j][lane];
            nib_pairs(w.x, &pb[j][0]);
            nib_pairs(w.y, &pb[j][4]);
            nib_pairs(w.z, &pb[j][8]);
            nib_pairs(w.w, &pb[j][12]);
            const int g = (j * 64 + lane) >> 1;
            ks_b[j] = bf16_to_f32(reinterpret_cast<const uint16_t*>(SB_.s)[g]);
            kc_b[j] = affine_c(ks_b[j], reinterpret_cast<const uint16_t*>(SB_.b)[g]);
        }
#pragma unroll
        for (int j = 0; j < SPL_B; ++j) {
#pragma unroll
            for (int i = 0; i < 16; ++i) pin(pb[j][i]);
            pin(ks_b[j]);
            pin(kc_b[j]);
        }
    };

    // lm_head streaming state: this wave's batches of LM_RPI rows, LM_NBUF
    // register buffers so that LM_NBUF - 1 batches are in flight while one is
    // reduced.  Rows: lm_full full rounds of LM_RPI-row batches (batch j of
    // wave gw: rows LM_RPI (gw + j W)), and the rest (fewer than a round) as
    // one short batch of at most ceil(rest / W) rows per wave, dealt
    // wave-major and taken first, so that its round trip overlaps the start
    // of the stream instead of adding a last round (a 31st round of whole
    // batches at vocab 248,320); its missing rows repeat its last row and
    // are not reported.
    constexpr int W = kNWG * kNCW;
    const int gw = wg * kNCW + cw;
    const int lm_full = p.vocab / (LM_RPI * W), lm_rest = p.vocab - lm_full * LM_RPI * W;
    const int lm_q = (lm_rest + W - 1) / W;
    const int lm_r0s = lm_full * LM_RPI * W + (cw * kNWG + wg) * lm_q;     // short batch
    const int lm_ns = lm_rest == 0 ? 0 : (p.vocab - lm_r0s < lm_q ? (p.vocab - lm_r0s > 0 ? p.vocab - lm_r0s : 0) : lm_q);
    const int lm_S = lm_ns > 0 ? 1 : 0;
    const int lm_rounds = lm_full + lm_S;
    auto lm_row0 = [&](int j) { return j < lm_S ? lm_r0s : LM_RPI * (gw + (j - lm_S) * W); };
    auto lm_nrows = [&](int j) { return j < lm_S ? lm_ns : LM_RPI; };
    struct LmBuf {
        uint4 w[LM_RPI];
        uint32_t s[LM_RPI], b[LM_RPI];
    };
    LmBuf lb[LM_NBUF];
    auto loadLM = [&](LmBuf& B, int round) {
        const int r0 = lm_row0(round), rl = r0 + lm_nrows(round) - 1;
#pragma unroll
        for (int r = 0; r < LM_RPI; ++r) {
            const int row = r0 + r < rl ? r0 + r : rl;
            B.w[r] = load_nt_u4(reinterpret_cast<const uint4*>(p.lm.wq + (int64_t)row * (H / 8)) + lane);
            B.s[r] = p.lm.s[(int64_t)row * (H / 64) + (lane >> 1)];
            B.b[r] = p.lm.b[(int64_t)row * (H / 64) + (lane >> 1)];
        }
    };

    // One layer; false if the step was aborted.  On entry this layer's gate
    // weights (this wave's own DMA) are issued and its up weights staged
    // (layer 0: issued by this wave too); its down weights are staged by B3.
    // (inlined twice: layer 0 is peeled, so that its copy waits for the
    // prologue's untracked DMA by exact counts, gate rows first)
    auto layer = [&](int l) __attribute__((always_inline)) -> bool {
        if (l == 0) {                                          // own gate and up DMA of the prologue
            wait_vmcnt<kDmaA / 2>();                           // gate rows (up rows still landing)
            unpackA(0);
            wait_vmcnt<0>();
            unpackA(1);
        } else {
            wait_vmcnt<0>();                                   // own gate-row DMA
            unpackA(0);                                        // while x is gathered
            unpackA(1);
        }
        lds_barrier();                                         // B1
        if (sm.abort) return false;
        if (l + 1 < L) dmaA(cw, l + 1, 0);                     // during the RMSNorm phase
        lds_barrier();                                         // B2
        // ---- gate/up rows rowA..rowA+RA-1 ----
        {
            uint32_t xp[16];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint4 c = sm.xp[w][lane];
                xp[4 * w] = c.x, xp[4 * w + 1] = c.y, xp[4 * w + 2] = c.z, xp[4 * w + 3] = c.w;
            }
            const float xs = sm.xs[lane];
            float acc[2 * RA + 2];   // value index v = r*2 + t; padded to 8 values
#pragma unroll
            for (int i = 0; i < 2 * RA + 2; ++i) acc[i] = 0.0f;
#pragma unroll
            for (int r = 0; r < RA; ++r)
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    acc[r * 2 + t] += affine_term_f(ks_a[t][r], kc_a[t][r], pairs_d(pa[t][r], xp), xs);
            const float v = wave_multi_reduce<8>(acc, lane);
            const float other = dpp_partner_f(v, 8);     // up partner (value index v^1, lane l^8)
            const int vidx = lane >> 3;
            if ((lane & 7) == 0 && (vidx & 1) == 0 && (vidx >> 1) < RA)
                sm.out[cw * RA + (vidx >> 1)] = swiglu_bf16(v, other);
        }
        lds_barrier();                                         // B3
        unpackB();                                             // while h is gathered
        lds_barrier();                                         // B4
        if (sm.abort) return false;
        // ---- down row rowB (+ residual) ----
        {
            // one partial per 64-slice third of K, reduced over the wave, then
            // added in order (the K-split order of the separate kernel)
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < SPL_B; ++j) {
                const int sl = j * 64 + lane;
                uint32_t hp[16];
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint4 c = sm.hp[w][sl];
                    hp[4 * w] = c.x, hp[4 * w + 1] = c.y, hp[4 * w + 2] = c.z, hp[4 * w + 3] = c.w;
                }
                acc[j] += affine_term_f(ks_b[j], kc_b[j], pairs_d(pb[j], hp), sm.hs[sl]);
            }
            const float v = wave_multi_reduce<4>(acc, lane);    // lane >> 4 = third
            const float v0 = lane_value(v, 0), v1 = lane_value(v, 16), v2 = lane_value(v, 32);
            float y = 0.0f;
            y += v0;
            y += v1;
            y += v2;
            if (lane == 0) {
                const int n = rowB;
                const uint32_t pair = sm.xraw[n >> 1];
                const float res = bf16_to_f32((n & 1) ? (pair >> 16) : (pair & 0xffffu));
                sm.out[cw] = f32_to_bf16(res + round_bf16(y));
            }
        }
        lds_barrier();                                         // B5
        return true;
    };

    bool aborted = L > 0 && !layer(0);
    for (int l = 1; l < L && !aborted; ++l)
        if (!layer(l)) aborted = true;

    // ---- lm_head + argmax over this wave's batches ----
    // (first two batches issued here, once the layer weights are dead, so they
    // are in flight during the exchange of the last hidden state)
    uint64_t best = 0;
    if (!aborted && p.vocab > 0) {
#pragma unroll
        for (int b = 0; b < LM_NBUF; ++b)
            if (b < lm_rounds) loadLM(lb[b], b);
        lds_barrier();                                         // B1 (x of the last layer)
        if (sm.abort) aborted = true;
    }
    if (!aborted && p.vocab > 0) {
        lds_barrier();                                         // B2 (final-normalized x)
        uint32_t xp[16];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint4 c = sm.xp[w][lane];
            xp[4 * w] = c.x, xp[4 * w + 1] = c.y, xp[4 * w + 2] = c.z, xp[4 * w + 3] = c.w;
        }
        const float xs = sm.xs[lane];
        auto consume = [&](LmBuf& B, int round) {
            float acc[LM_RPI];
#pragma unroll
            for (int r = 0; r < LM_RPI; ++r) {
                acc[r] = 0.0f;
                acc[r] += affine_term(B.s[r], B.b[r], slice_d(B.w[r], xp), xs);
            }
            if (round + LM_NBUF < lm_rounds) loadLM(B, round + LM_NBUF);   // refill LM_NBUF rounds ahead
            const float v = wave_multi_reduce<LM_RPI>(acc, lane);
            constexpr int SHL = 6 - log2_const<LM_RPI>();
            const int row = lm_row0(round) + (lane >> SHL);
            if ((lane & ((1 << SHL) - 1)) == 0 && (lane >> SHL) < lm_nrows(round)) {
                const uint64_t key = argmax_key(f32_to_bf16(v), (uint32_t)row);
                best = key > best ? key : best;
            }
        };
        for (int round = 0; round < lm_rounds; round += LM_NBUF) {
#pragma unroll
            for (int b = 0; b < LM_NBUF; ++b)
                if (round + b < lm_rounds) consume(lb[b], round + b);
        }
    }
    best = wave_max_u64(best);
    if (lane == 0) sm.best[cw] = best;
    lds_barrier();                                             // B6
}

}  // namespace dec

// Co-residency of the 256 workgroups, checked once per device.
constexpr int kMaxDecDevices = 64;
static int g_dec_ok[kMaxDecDevices];
static bool g_dec_checked[kMaxDecDevices];
static std::mutex g_dec_mu;

// Poll iterations before a wait gives up (each iteration is one round trip
// to L2 plus a short sleep, about 1 us): about a second.
constexpr int kSpinLimit = 1 << 20;

}  // namespace mq4

using namespace mq4;

extern "C" size_t mq4_decode_workspace_size(int64_t hidden, int64_t intermediate, int64_t vocab) {
    (void)vocab;
    if (hidden != dec::H || intermediate != dec::I) return 0;
    // ctrl (256 B) + copies of the x and h words + per-workgroup partial
    // keys, each 256-byte aligned
    const size_t xw = (size_t)dec::kCopies * hidden / 2 * 8, hw = (size_t)dec::kCopies * intermediate / 2 * 8;
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    return 256 + up(xw) + up(hw) + up((size_t)dec::kNWG * 8);
}

extern "C" int mq4_decode_step(const uint16_t* x_in, int64_t hidden, int64_t intermediate, int64_t n_layers,
                               const mq4_mlp_layer* layers, const uint16_t* final_norm, float eps,
                               const uint32_t* lm_wq, const uint16_t* lm_scales, const uint16_t* lm_biases,
                               int64_t vocab, uint32_t* idx, uint16_t* x_out, void* workspace,
                               size_t workspace_bytes, void* stream) {
    const char* what = "mq4_decode_step";
    if (hidden != dec::H || intermediate != dec::I)
        return fail(MQ4_ERR_UNSUPPORTED, "%s: built for hidden=%d, intermediate=%d (got %lld, %lld)", what, dec::H,
                    dec::I, (long long)hidden, (long long)intermediate);
    if (n_layers < 0 || n_layers > dec::kMaxLayers)
        return fail(MQ4_ERR_UNSUPPORTED, "%s: n_layers must be in [0, %d]", what, dec::kMaxLayers);
    if (vocab < 0 || vocab > (1LL << 30))
        return fail(MQ4_ERR_INVALID_ARG, "%s: vocab must be in [0, 2^30]", what);
    if (vocab == 0 && n_layers == 0)
        return fail(MQ4_ERR_INVALID_ARG, "%s: nothing to do (no layers and vocab 0)", what);
    if (!x_in || (n_layers > 0 && !layers))
        return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer", what);
    if (vocab > 0 && (!final_norm || !lm_wq || !lm_scales || !lm_biases || !idx))
        return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer (final norm, lm_head or idx)", what);
    if (!aligned(x_in, 16) || (x_out && !aligned(x_out, 4)) ||
        (vocab > 0 && (!aligned(final_norm, 16) || !aligned(lm_wq, 16))))
        return fail(MQ4_ERR_ALIGNMENT, "%s: x_in, norms and packed weights must be 16-byte aligned", what);
    const size_t need = mq4_decode_workspace_size(hidden, intermediate, vocab);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
        return fail(MQ4_ERR_WORKSPACE, "%s: workspace needs %zu bytes, 256-byte aligned, zero-filled once", what,
                    need);
    dec::Params p{};
    for (int64_t l = 0; l < n_layers; ++l) {
        const mq4_mlp_layer& s = layers[l];
        if (!s.norm_weight || !s.gate_wq || !s.gate_scales || !s.gate_biases || !s.up_wq || !s.up_scales ||
            !s.up_biases || !s.down_wq || !s.down_scales || !s.down_biases)
            return fail(MQ4_ERR_INVALID_ARG, "%s: null pointer in layer %lld", what, (long long)l);
        if (!aligned(s.norm_weight, 16) || !aligned(s.gate_wq, 16) || !aligned(s.up_wq, 16) ||
            !aligned(s.down_wq, 16))
            return fail(MQ4_ERR_ALIGNMENT, "%s: layer %lld norm and packed weights must be 16-byte aligned", what,
                        (long long)l);
        if (!aligned(s.gate_scales, 4) || !aligned(s.gate_biases, 4) || !aligned(s.up_scales, 4) ||
            !aligned(s.up_biases, 4) || !aligned(s.down_scales, 4) || !aligned(s.down_biases, 4))
            return fail(MQ4_ERR_ALIGNMENT, "%s: layer %lld scales and biases must be 4-byte aligned", what,
                        (long long)l);
        p.layers[l] = {s.norm_weight,
                       {s.gate_wq, s.gate_scales, s.gate_biases},
                       {s.up_wq, s.up_scales, s.up_biases},
                       {s.down_wq, s.down_scales, s.down_biases}};
    }
    {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDecDevices)
            return fail(MQ4_ERR_HIP, "%s: hipGetDevice failed", what);
        std::lock_guard<std::mutex> lk(g_dec_mu);
        if (!g_dec_checked[dev]) {
            int cus = 0, occ = 0;
            if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, dec::decode_step_kernel, dec::kThreads, 0) !=
                    hipSuccess)
                return fail(MQ4_ERR_HIP, "%s: device query failed", what);
            g_dec_ok[dev] = (cus >= dec::kNWG && occ >= 1) ? 1 : 0;
            g_dec_checked[dev] = true;
        }
        if (g_dec_ok[dev] == 0)
            return fail(MQ4_ERR_UNSUPPORTED, "%s: needs %d co-resident workgroups of %d threads", what, dec::kNWG,
                        dec::kThreads);
    }
    p.x_in = x_in;
    p.x_out = x_out;
    p.idx = idx;
    p.final_norm = final_norm;
    p.eps = eps;
    p.lm = {lm_wq, lm_scales, lm_biases};
    p.vocab = (int)vocab;
    p.n_layers = (int)n_layers;
    char* ws = reinterpret_cast<char*>(workspace);
    const size_t xw = ((size_t)dec::kCopies * hidden / 2 * 8 + 255) / 256 * 256,
                 hw = ((size_t)dec::kCopies * intermediate / 2 * 8 + 255) / 256 * 256;
    p.ctrl = reinterpret_cast<uint32_t*>(ws);
    p.xbuf = reinterpret_cast<uint64_t*>(ws + 256);
    p.hbuf = reinterpret_cast<uint64_t*>(ws + 256 + xw);
    p.part = reinterpret_cast<uint64_t*>(ws + 256 + xw + hw);
    p.spin_limit = kSpinLimit;
    hipLaunchKernelGGL(dec::decode_step_kernel, dim3(dec::kNWG), dim3(dec::kThreads), 0, as_stream(stream), p);
    return launch_status(what);
}
