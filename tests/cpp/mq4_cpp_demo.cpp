// C++ caller of libmq4 through marlin-mlx_amd/csrc/mq4.hpp, shaped like the
// reference's decode step (src/model/marlin.cpp:110-145, 161-169): quantize
// two synthetic layers and an lm_head, run hidden += mlp(rms_norm(hidden))
// twice, then the greedy lm_head.  Prints the token and the final hidden
// state's bf16 words so a test can compare them with the Python binding.
// With a path argument the lm_head also makes a round trip through the
// on-disk Q4 cache (mq4_cache.hpp) and the greedy head uses the loaded copy.
#include <cstdio>
#include <vector>

#include "mq4.hpp"
#include "mq4_cache.hpp"

#define CHECK(r)                                                                    \
    do {                                                                            \
        auto&& r_ = (r);                                                            \
        if (!r_) {                                                                  \
            std::fprintf(stderr, "error %d: %s\n", r_.error().code, r_.error().message.c_str()); \
            return 1;                                                               \
        }                                                                           \
    } while (0)

static int fill(uint16_t* p, int64_t n, uint64_t sid, double mu, double sigma, hipStream_t st) {
    return mq4_fill_normal_bf16(p, n, 0x4D41524Cull, sid, mu, sigma, 0, st);
}

int main(int argc, char** argv) {
    const int64_t H = 512, I = 1024, V = 4096, LAYERS = 2;
    hipStream_t st;
    if (hipStreamCreate(&st) != hipSuccess) return 2;
    mq4::DeviceBuffer wtmp(2 * I * H > 2 * V * H ? 2 * I * H : 2 * V * H);
    std::vector<mq4::MLPWeights> layers(LAYERS);
    std::vector<mq4::DeviceBuffer> norms;
    // the layers' bf16 weights, then one batched quantize of all of them
    // (the loader loop of src/model/weights.cpp:147-160)
    std::vector<mq4::DeviceBuffer> raw;
    std::vector<mq4::WeightView> views;
    for (int l = 0; l < LAYERS; ++l) {
        const int64_t shp[3][2] = {{I, H}, {I, H}, {H, I}};
        for (int p = 0; p < 3; ++p) {
            raw.emplace_back((size_t)(2 * shp[p][0] * shp[p][1]));
            if (fill(raw.back().as<uint16_t>(), shp[p][0] * shp[p][1], 1000 + 3 * l + p, 0.0, 0.02, st)) return 3;
            views.push_back({raw.back().as<uint16_t>(), shp[p][0], shp[p][1]});
        }
        norms.emplace_back(2 * H);
        if (fill(norms.back().as<uint16_t>(), H, 2100 + l, 0.1, 0.02, st)) return 3;
    }
    {
        auto qs = mq4::quantize_weights(views, st);
        CHECK(qs);
        for (int l = 0; l < LAYERS; ++l) {
            layers[l].gate_proj = std::move(qs.value()[3 * l]);
            layers[l].up_proj = std::move(qs.value()[3 * l + 1]);
            layers[l].down_proj = std::move(qs.value()[3 * l + 2]);
        }
    }
    if (fill(wtmp.as<uint16_t>(), V * H, 2000, 0.0, 0.02, st)) return 3;
    auto lmq = mq4::quantize_weight(wtmp.as<uint16_t>(), V, H, st);
    CHECK(lmq);
    if (argc > 1) {   // save the quantized lm_head and continue with the copy loaded back
        if (hipStreamSynchronize(st) != hipSuccess) return 4;
        CHECK(mq4::save_q4_cache(argv[1], {{"lm_head", &lmq.value()}}));
        auto loaded = mq4::load_q4_cache(argv[1]);
        CHECK(loaded);
        auto it = loaded.value().find("lm_head");
        if (it == loaded.value().end()) return 5;
        lmq.value() = std::move(it->second);
    }
    mq4::DeviceBuffer final_norm(2 * H), hidden(2 * H), hidden2(2 * H), h(2 * I), idx(4), logits(2 * V), sidx(8);
    if (fill(final_norm.as<uint16_t>(), H, 2001, 0.1, 0.02, st)) return 3;
    if (fill(hidden.as<uint16_t>(), H, 3000, 0.0, 1.0, st)) return 3;
    if (fill(hidden2.as<uint16_t>(), H, 3000, 0.0, 1.0, st)) return 3;
    mq4::MlpResidual mlp(1, H, I);
    for (int l = 0; l < LAYERS; ++l) {
        CHECK(mq4::mlp_forward_residual(hidden.as<uint16_t>(), 1, norms[l].as<uint16_t>(), 1e-6f, layers[l],
                                        h.as<uint16_t>(), st));
        CHECK(mlp(hidden2.as<uint16_t>(), 1, norms[l].as<uint16_t>(), 1e-6f, layers[l], st));   // one call
    }
    mq4::GreedyLmHead head(1, V);
    CHECK(head(hidden.as<uint16_t>(), 1, final_norm.as<uint16_t>(), 1e-6f, lmq.value(), idx.as<uint32_t>(),
               logits.as<uint16_t>(), st));
    // sample_token on the same logits: temperature 0.8, top-k 50 (seed 5),
    // then the greedy case (temperature 0), which must give the argmax token
    mq4::Sampler sampler(1, V);
    mq4::SamplingConfig cfg;
    cfg.temperature = 0.8f;
    cfg.top_k = 50;
    cfg.seed = 5;
    CHECK(sampler(logits.as<uint16_t>(), 1, cfg, sidx.as<uint32_t>(), nullptr, st));
    cfg.temperature = 0.0f;
    CHECK(sampler(logits.as<uint16_t>(), 1, cfg, sidx.as<uint32_t>() + 1, nullptr, st));
    if (hipStreamSynchronize(st) != hipSuccess) return 4;
    uint32_t stok[2] = {0, 0};
    if (hipMemcpy(stok, sidx.get(), 8, hipMemcpyDeviceToHost) != hipSuccess) return 4;
    uint32_t tok = 0;
    std::vector<uint16_t> hid(H), hid2(H);
    if (hipMemcpy(&tok, idx.get(), 4, hipMemcpyDeviceToHost) != hipSuccess) return 4;
    if (hipMemcpy(hid.data(), hidden.get(), 2 * H, hipMemcpyDeviceToHost) != hipSuccess) return 4;
    if (hipMemcpy(hid2.data(), hidden2.get(), 2 * H, hipMemcpyDeviceToHost) != hipSuccess) return 4;
    std::printf("token %u\nhidden", tok);
    for (int64_t i = 0; i < H; ++i) std::printf(" %u", hid[i]);
    std::printf("\nsampled %u greedy %u\n", stok[0], stok[1]);
    std::printf("mlp_residual_same %d\n", hid == hid2 ? 1 : 0);
    // zero rows: every mirror returns success without touching its outputs
    bool empty_ok = mq4::qmatmul(hidden.as<uint16_t>(), 0, lmq.value(), logits.as<uint16_t>(), st).ok() &&
                    mq4::mlp_forward_residual(hidden.as<uint16_t>(), 0, norms[0].as<uint16_t>(), 1e-6f, layers[0],
                                              h.as<uint16_t>(), st).ok() &&
                    mlp(hidden2.as<uint16_t>(), 0, norms[0].as<uint16_t>(), 1e-6f, layers[0], st).ok() &&
                    head(hidden.as<uint16_t>(), 0, final_norm.as<uint16_t>(), 1e-6f, lmq.value(), idx.as<uint32_t>(),
                         nullptr, st).ok();
    std::printf("empty_ok %d\n", empty_ok ? 1 : 0);

    // MlpResidual sized for 40 rows serves every row count up to 40 (24 and
    // 32 rows need the two fp32 K parts of the MFMA path, more per row than
    // the paired GEMM operands of 33-40 rows); below 33 rows it gives the
    // separate entries' bits
    bool rows_ok = true;
    {
        const int64_t R = 40;
        mq4::DeviceBuffer xa(2 * R * H), xb(2 * R * H), hb(2 * R * I);
        mq4::MlpResidual mlp40(R, H, I);
        for (int64_t M : {24, 32, 40}) {
            if (fill(xa.as<uint16_t>(), M * H, 3100, 0.0, 1.0, st)) return 3;
            if (fill(xb.as<uint16_t>(), M * H, 3100, 0.0, 1.0, st)) return 3;
            auto r = mlp40(xa.as<uint16_t>(), M, norms[0].as<uint16_t>(), 1e-6f, layers[0], st);
            if (!r) {
                std::fprintf(stderr, "MlpResidual(40 rows) at M=%lld: %s\n", (long long)M, r.error().message.c_str());
                rows_ok = false;
                continue;
            }
            CHECK(mq4::mlp_forward_residual(xb.as<uint16_t>(), M, norms[0].as<uint16_t>(), 1e-6f, layers[0],
                                            hb.as<uint16_t>(), st));
            if (hipStreamSynchronize(st) != hipSuccess) return 4;
            if (M < 33) {
                std::vector<uint16_t> a(M * H), b(M * H);
                if (hipMemcpy(a.data(), xa.get(), 2 * M * H, hipMemcpyDeviceToHost) != hipSuccess ||
                    hipMemcpy(b.data(), xb.get(), 2 * M * H, hipMemcpyDeviceToHost) != hipSuccess)
                    return 4;
                rows_ok = rows_ok && a == b;
            }
        }
    }
    std::printf("mlp_residual_rows_ok %d\n", rows_ok ? 1 : 0);

    // another format (group 128, or 2 bits) is refused before any launch
    bool rejected = true;
    {
        mq4::MLPWeights odd;
        odd.gate_proj.quantized = odd.up_proj.quantized = odd.down_proj.quantized = true;
        odd.gate_proj.group_size = 128;
        auto r = mlp(hidden2.as<uint16_t>(), 1, norms[0].as<uint16_t>(), 1e-6f, odd, st);
        rejected = rejected && !r && r.error().code == MQ4_ERR_UNSUPPORTED;
        auto r2 = mq4::mlp_forward_residual(hidden.as<uint16_t>(), 1, norms[0].as<uint16_t>(), 1e-6f, odd,
                                            h.as<uint16_t>(), st);
        rejected = rejected && !r2 && r2.error().code == MQ4_ERR_UNSUPPORTED;
        mq4::QuantizedTensor two_bit;
        two_bit.quantized = true;
        two_bit.bits = 2;
        auto r3 = head(hidden.as<uint16_t>(), 1, final_norm.as<uint16_t>(), 1e-6f, two_bit, idx.as<uint32_t>(),
                       nullptr, st);
        rejected = rejected && !r3 && r3.error().code == MQ4_ERR_UNSUPPORTED;
    }
    std::printf("format_rejected %d\n", rejected ? 1 : 0);

    // mq4::BatchedMlpLayers (one launch per layer, hidden 2048 / intermediate
    // 6144): two layers over 16 rows as one call equal the two one-layer
    // calls chained by the caller, bit for bit; more rows than the workspace
    // was sized for are refused
    bool batched_ok = true;
    {
        const int64_t BH = 2048, BI = 6144, R = 16;
        std::vector<mq4::DeviceBuffer> braw;
        std::vector<mq4::WeightView> bviews;
        std::vector<mq4::MLPWeights> bl(2);
        std::vector<mq4::DeviceBuffer> bnorm;
        for (int l = 0; l < 2; ++l) {
            const int64_t shp[3][2] = {{BI, BH}, {BI, BH}, {BH, BI}};
            for (int q = 0; q < 3; ++q) {
                braw.emplace_back((size_t)(2 * shp[q][0] * shp[q][1]));
                if (fill(braw.back().as<uint16_t>(), shp[q][0] * shp[q][1], 5000 + 3 * l + q, 0.0, 0.02, st)) return 3;
                bviews.push_back({braw.back().as<uint16_t>(), shp[q][0], shp[q][1]});
            }
            bnorm.emplace_back(2 * BH);
            if (fill(bnorm.back().as<uint16_t>(), BH, 5100 + l, 0.1, 0.02, st)) return 3;
        }
        auto qs = mq4::quantize_weights(bviews, st);
        CHECK(qs);
        for (int l = 0; l < 2; ++l) {
            bl[l].gate_proj = std::move(qs.value()[3 * l]);
            bl[l].up_proj = std::move(qs.value()[3 * l + 1]);
            bl[l].down_proj = std::move(qs.value()[3 * l + 2]);
        }
        mq4::BatchedMlpLayers stack({{bnorm[0].as<uint16_t>(), &bl[0]}, {bnorm[1].as<uint16_t>(), &bl[1]}}, R);
        mq4::DeviceBuffer x0(2 * R * BH), x1(2 * R * BH), x2(2 * R * BH), xs(2 * R * BH);
        if (fill(x0.as<uint16_t>(), R * BH, 5200, 0.0, 1.0, st)) return 3;
        CHECK(stack(x0.as<uint16_t>(), R, 1e-6f, xs.as<uint16_t>(), st));               // both layers
        CHECK(stack(x0.as<uint16_t>(), R, 1e-6f, x1.as<uint16_t>(), st, 0, 1));         // layer 0
        CHECK(stack(x1.as<uint16_t>(), R, 1e-6f, x2.as<uint16_t>(), st, 1, 1));         // layer 1
        if (hipStreamSynchronize(st) != hipSuccess) return 4;
        std::vector<uint16_t> a(R * BH), b(R * BH);
        if (hipMemcpy(a.data(), xs.get(), 2 * R * BH, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(b.data(), x2.get(), 2 * R * BH, hipMemcpyDeviceToHost) != hipSuccess)
            return 4;
        batched_ok = a == b;
        auto over = stack(x0.as<uint16_t>(), R + 1, 1e-6f, xs.as<uint16_t>(), st);
        batched_ok = batched_ok && !over && over.error().code == MQ4_ERR_WORKSPACE;
    }
    std::printf("batched_layers_ok %d\n", batched_ok ? 1 : 0);
    (void)hipStreamDestroy(st);
    return 0;
}
