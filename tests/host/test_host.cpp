// Tests of the C++17 host layer (sam.cpp_amd/host/sam_hip.hpp).
//   test_host --cpu : options, CLI flags, format policy, status mapping and
//                     the no-device behaviour (no GPU needed)
//   test_host --gpu : HipBackend + HipGraphExecution on device 0, products
//                     checked against the oracle's native CPU path
// Cases follow the reference's own option, CLI and policy tests
// (tests/api/test_contracts.cpp:327-339, tests/models/test_image_cli.cpp:25-65,
// tests/runtime/ggml/test_quantization.cpp:105-175), extended to HIP.
#include "sam_hip.hpp"
#include "feature_cache.hpp"
#include "ggml_oracle.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

namespace {

int g_failures = 0;
int g_checks = 0;

#define CHECK(cond)                                                                   \
    do {                                                                              \
        ++g_checks;                                                                   \
        if (!(cond)) {                                                                \
            ++g_failures;                                                             \
            std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
        }                                                                             \
    } while (0)

template <class E>
bool throws(const std::function<void()>& f, const char* needle = nullptr) {
    try {
        f();
    } catch (const E& e) {
        return !needle || std::strstr(e.what(), needle) != nullptr;
    } catch (...) {
        return false;
    }
    return false;
}

void test_options() {
    using namespace sam;
    BackendOptions o;
    validate_backend_options(o);
    o.backend = Backend::Hip;
    o.hip_device = 3;
    o.hip_compute = HipComputeMode::F16;
    validate_backend_options(o);
    CHECK(throws<std::invalid_argument>([] {
        BackendOptions b;
        b.hip_device = 1;   // needs --backend hip
        validate_backend_options(b);
    }, "explicit HIP backend"));
    CHECK(throws<std::invalid_argument>([] {
        BackendOptions b;
        b.backend = Backend::Hip;
        b.hip_device = -1;
        validate_backend_options(b);
    }));
    CHECK(throws<std::invalid_argument>([] {
        BackendOptions b;
        b.hip_compute = HipComputeMode::F16;
        validate_backend_options(b);
    }, "explicit HIP backend"));
    CHECK(throws<std::invalid_argument>([] {
        BackendOptions b;
        b.backend = Backend::Hip;
        b.cuda_device = 1;   // CUDA rules are unchanged
        validate_backend_options(b);
    }, "CUDA device"));
    CHECK(throws<std::invalid_argument>([] {
        BackendOptions b;
        b.backend = Backend::Hip;
        b.cpu_compute = CpuComputeMode::NativeQuantized;
        validate_backend_options(b);
    }));
    CHECK(throws<std::invalid_argument>([] {
        BackendOptions b;
        b.backend = static_cast<Backend>(17);
        validate_backend_options(b);
    }, "unknown SAM backend"));
    CHECK(throws<std::invalid_argument>([] {
        BackendOptions b;
        b.threads = 0;
        validate_backend_options(b);
    }));
}

void test_flags() {
    using namespace sam;
    auto parse = [](std::vector<std::pair<std::string, std::string>> args) {
        BackendOptions o;
        std::vector<std::string> seen;
        for (auto& a : args)
            if (!parse_backend_flag(a.first, a.second, o, seen)) throw std::invalid_argument("unowned " + a.first);
        finish_backend_flags(o, seen);
        return o;
    };
    const BackendOptions o = parse({{"--backend", "hip"}, {"--hip-device", "2"}, {"--hip-compute", "f16"}});
    CHECK(o.backend == Backend::Hip && o.hip_device == 2 && o.hip_compute == HipComputeMode::F16);
    CHECK(std::string(backend_name(o.backend)) == "hip");
    CHECK(parse({{"--backend", "hip"}}).hip_compute == HipComputeMode::Q8Native);
    CHECK(throws<std::invalid_argument>([&] { parse({{"--hip-device", "1"}}); }, "--hip-device requires --backend hip"));
    CHECK(throws<std::invalid_argument>([&] { parse({{"--hip-compute", "f16"}}); }, "--hip-compute requires"));
    CHECK(throws<std::invalid_argument>([&] { parse({{"--backend", "rocm"}}); }, "--backend must be"));
    CHECK(throws<std::invalid_argument>([&] { parse({{"--backend", "hip"}, {"--hip-device", "-1"}}); }));
    CHECK(throws<std::invalid_argument>([&] { parse({{"--backend", "hip"}, {"--hip-device", "1x"}}); }));
    CHECK(throws<std::invalid_argument>([&] { parse({{"--backend", "hip"}, {"--hip-compute", "f32"}}); }));
    BackendOptions unused;
    std::vector<std::string> seen;
    CHECK(!parse_backend_flag("--score-threshold", "0.5", unused, seen));
}

void test_policy() {
    using namespace sam::policy;
    CHECK(is_image_quantized_linear_weight("vit.blocks.0.attn.qkv.weight", false));
    CHECK(is_image_quantized_linear_weight("vit.blocks.31.mlp.lin2.weight", false));
    CHECK(!is_image_quantized_linear_weight("vit.blocks.32.mlp.lin2.weight", false));
    CHECK(!is_image_quantized_linear_weight("vit.blocks.01.mlp.lin2.weight", false));
    CHECK(!is_image_quantized_linear_weight("vit.blocks.0.attn.qkv.bias", false));
    CHECK(!is_image_quantized_linear_weight("text.blocks.3.mlp.fc1.weight", false));
    CHECK(is_image_quantized_linear_weight("text.blocks.3.mlp.fc1.weight", true));
    CHECK(!is_image_quantized_linear_weight("text.blocks.24.mlp.fc1.weight", true));
    CHECK(is_image_q8_k_fallback_weight("vit.blocks.7.mlp.lin2.weight"));
    CHECK(!is_image_q8_k_fallback_weight("vit.blocks.7.mlp.lin1.weight"));

    const auto* q4 = image_quantization_profile("image-linear-q4_k-v1");
    const auto* vq8 = image_quantization_profile("image-vision-linear-q8_0-v1");
    CHECK(q4 && q4->type == SAMHIP_TYPE_Q4_K && q4->file_type == 14 && q4->quantize_text_linear);
    CHECK(vq8 && vq8->type == SAMHIP_TYPE_Q8_0 && !vq8->quantize_text_linear);
    CHECK(!image_quantization_profile("image-linear-q3_k-v1"));
    CHECK(image_quantized_tensor_type("vit.blocks.4.mlp.lin2.weight", {4736, 1024}, *q4) == SAMHIP_TYPE_Q8_0);
    CHECK(image_quantized_tensor_type("vit.blocks.4.mlp.lin1.weight", {1024, 4736}, *q4) == SAMHIP_TYPE_Q4_K);
    CHECK(image_quantized_tensor_type("vit.blocks.4.attn.qkv.weight", {1024, 3072}, *vq8) == SAMHIP_TYPE_Q8_0);
    CHECK(image_quantized_tensor_type("text.blocks.0.mlp.fc2.weight", {4096, 1024}, *vq8) == SAMHIP_TYPE_F32);
    CHECK(image_quantized_tensor_type("text.blocks.0.mlp.fc2.weight", {4096, 1024}, *q4) == SAMHIP_TYPE_Q4_K);
    CHECK(throws<std::runtime_error>([&] { image_quantized_tensor_type("vit.blocks.4.attn.qkv.weight", {1000, 3072}, *q4); },
                                     "noncanonical row width"));
    // test_quantization.cpp:105-166 cases
    const auto* q6 = image_quantization_profile("image-linear-q6_k-v1");
    CHECK(!image_quantization_profile("q4_k"));
    CHECK(image_quantized_tensor_type("vit.blocks.0.mlp.lin2.weight", {4736, 1024}, *q6) == SAMHIP_TYPE_Q8_0);
    CHECK(image_quantized_tensor_type("vit.blocks.0.mlp.lin2.weight", {4864, 1024}, *q6) == SAMHIP_TYPE_Q6_K);
    CHECK(throws<std::runtime_error>([&] { image_quantized_tensor_type("vit.blocks.0.attn.qkv.weight", {4736, 3072}, *q6); }));
    CHECK(image_quantized_tensor_type("vit.blocks.32.attn.qkv.weight", {1024, 3072}, *q4) == SAMHIP_TYPE_F32);
    CHECK(image_quantized_tensor_type("vit.blocks.0.mlp.lin2.bias", {1024}, *q4) == SAMHIP_TYPE_F32);
    CHECK(image_quantized_tensor_type("neck.det.0.conv_1x1.weight", {256, 256, 1, 1}, *vq8) == SAMHIP_TYPE_F32);

    const auto* m6 = modular_image_quantization_profile("image-full-linear-q6_k-v1");
    const auto* m8 = modular_image_quantization_profile("image-modules-linear-q8_0-v1");
    CHECK(m6 && m6->type == SAMHIP_TYPE_Q6_K && m6->file_type == 18 && m6->full_preset);
    CHECK(m8 && m8->type == SAMHIP_TYPE_Q8_0 && !m8->full_preset);
    const std::vector<std::string> all{"vision", "text", "fusion", "decoder"};
    CHECK(image_modular_quantized_tensor_type("ddec.layers.5.ca_text.in_proj_weight", {256, 768}, *m6, all) == SAMHIP_TYPE_Q6_K);
    CHECK(image_modular_quantized_tensor_type("ddec.layers.6.ca_text.in_proj_weight", {256, 768}, *m6, all) == SAMHIP_TYPE_F32);
    CHECK(image_modular_quantized_tensor_type("fenc.layers.2.linear2.weight", {2048, 256}, *m6, all) == SAMHIP_TYPE_Q6_K);
    CHECK(image_modular_quantized_tensor_type("fenc.layers.2.linear2.weight", {2048, 256}, *m6, {"vision"}) == SAMHIP_TYPE_F32);
    CHECK(image_modular_quantized_tensor_type("text.resizer.weight", {1024, 256}, *m8, {"text"}) == SAMHIP_TYPE_Q8_0);
    CHECK(image_modular_quantized_tensor_type("vit.blocks.1.mlp.lin2.weight", {4736, 1024}, *m6, all) == SAMHIP_TYPE_Q8_0);
    CHECK(image_modular_quantized_tensor_type("geom.final_proj.weight", {256, 256}, *m6, all) == SAMHIP_TYPE_Q6_K);
    CHECK(image_modular_quantized_tensor_type("ddec.boxRPB_embed_y.layers.1.weight", {256, 2}, *m8, all) == SAMHIP_TYPE_Q8_0);
    CHECK(image_modular_quantized_tensor_type("ddec.boxRPB_embed_y.layers.2.weight", {256, 2}, *m8, all) == SAMHIP_TYPE_F32);
    CHECK(image_modular_quantized_tensor_type("seg.mask_predictor.mask_embed.layers.2.weight", {256, 256}, *m8, all) ==
          SAMHIP_TYPE_Q8_0);
    // widths that hold no whole K-quant super-block stay F32, Q8_0 needs 32
    CHECK(image_modular_quantized_tensor_type("ddec.bbox_embed.layers.2.weight", {160, 4}, *m6, all) == SAMHIP_TYPE_F32);
    CHECK(image_modular_quantized_tensor_type("ddec.bbox_embed.layers.2.weight", {160, 4}, *m8, all) == SAMHIP_TYPE_Q8_0);
    CHECK(image_modular_quantized_tensor_type("ddec.bbox_embed.layers.2.weight", {100, 4}, *m8, all) == SAMHIP_TYPE_F32);
    CHECK(image_modular_quantized_tensor_type("vit.blocks.1.mlp.lin2.weight", {4736, 1024, 1}, *m6, all) == SAMHIP_TYPE_F32);

    CHECK(parse_image_quantization_modules("vision,fusion") == (std::vector<std::string>{"vision", "fusion"}));
    CHECK(throws<std::runtime_error>([] { parse_image_quantization_modules(""); }, "empty"));
    CHECK(throws<std::runtime_error>([] { parse_image_quantization_modules("text,vision"); }, "canonical"));
    CHECK(throws<std::runtime_error>([] { parse_image_quantization_modules("vision,vision"); }, "canonical"));
    CHECK(throws<std::runtime_error>([] { parse_image_quantization_modules("vision,"); }, "canonical"));
    CHECK(throws<std::runtime_error>([] { parse_image_quantization_modules(",vision"); }, "canonical"));
    CHECK(throws<std::runtime_error>([] { parse_image_quantization_modules("vision,,text"); }, "canonical"));
    CHECK(throws<std::runtime_error>([] { parse_image_quantization_modules("Vision"); }, "canonical"));
    CHECK(throws<std::runtime_error>([] { parse_image_quantization_modules("vision text"); }, "canonical"));
    CHECK(throws<std::runtime_error>([] { parse_image_quantization_modules("decoder,fusion"); }, "canonical"));
    CHECK(parse_image_quantization_modules("vision,text,fusion,decoder") ==
          (std::vector<std::string>{"vision", "text", "fusion", "decoder"}));
    CHECK(parse_image_quantization_modules("decoder") == (std::vector<std::string>{"decoder"}));
    CHECK(parse_image_quantization_modules("text,decoder") == (std::vector<std::string>{"text", "decoder"}));
}

void test_status_mapping_without_device() {
    using namespace sam;
    // invalid argument maps to std::invalid_argument, with the library's message
    CHECK(throws<std::invalid_argument>([] { check_status(samhip_mul_mat(nullptr, nullptr, nullptr, nullptr)); },
                                        "null context"));
    CHECK(throws<std::runtime_error>([] { check_status(SAMHIP_ERR_DEVICE); }));
    samhip_tensor w = make_tensor(SAMHIP_TYPE_Q4_K, 1000, 8, 144, 576, reinterpret_cast<void*>(256));
    samhip_tensor x = make_tensor(SAMHIP_TYPE_F32, 1000, 4, 4, 4000, reinterpret_cast<void*>(256));
    samhip_tensor y = make_tensor(SAMHIP_TYPE_F32, 8, 4, 4, 32, reinterpret_cast<void*>(256));
    CHECK(!HipBackend::supports_mul_mat(w, x, y));   // 1000 is not a multiple of 256
    // a graph with that node fails in prepare, naming node and sources
    HipGraphExecution graph(nullptr);
    graph.add({HipOp::MulMat, "vit.blocks.0.mlp.lin1", {"vit.blocks.0.mlp.lin1.weight", "x"}, {w, x}, y});
    CHECK(throws<std::runtime_error>([&] { graph.prepare(); },
                                     "no backend supports SAM operation MUL_MAT tensor vit.blocks.0.mlp.lin1 "
                                     "source0=vit.blocks.0.mlp.lin1.weight/q4_K source1=x/f32"));
}

void test_no_device() {
    int n = -1;
    sam::check_status(samhip_device_count(&n));
    if (n != 0) return;
    CHECK(throws<std::runtime_error>([] { sam::HipBackend::make(0); }, "no visible devices"));
}

// Feature-cache snapshots without a device: the reference's HostTensor
// checks (src/runtime/ggml/host_tensor.hpp:36-91).
void test_feature_cache_cpu() {
    using namespace sam;
    // exact host decode of hand-made Q8_0 blocks: d = 0.5, codes -3 and 127
    std::vector<uint8_t> blk(34, 0);
    blk[0] = 0x00;
    blk[1] = 0x38;   // 0.5 in binary16
    blk[2] = uint8_t(int8_t(-3));
    blk[33] = 127;
    std::vector<uint8_t> two = blk;
    two.insert(two.end(), blk.begin(), blk.end());
    const HipHostTensor q = HipHostTensor::from_bytes(SAMHIP_TYPE_Q8_0, 1, 64, two);
    const std::vector<float> f = q.as_f32();
    CHECK(f.size() == 64 && f[0] == -1.5f && f[1] == 0.f && f[31] == 63.5f && f[32] == -1.5f && f[63] == 63.5f);
    // flattening allowed, a different row layout is not
    q.validate_shape(64, 1, 1, 1);
    CHECK(throws<std::invalid_argument>([&] { q.validate_shape(32, 2, 1, 1); }, "row layout"));
    CHECK(throws<std::invalid_argument>([&] { q.validate_shape(64, 2, 1, 1); }, "row layout"));
    CHECK(throws<std::invalid_argument>([&] { q.validate_shape(64, 0, 1, 1); }, "dimension"));
    // non-finite or negative scales are rejected
    for (uint16_t bad : {uint16_t(0x7c00), uint16_t(0x7e00), uint16_t(0xb800)}) {
        std::vector<uint8_t> b = two;
        b[34] = uint8_t(bad & 0xff);
        b[35] = uint8_t(bad >> 8);
        CHECK(throws<std::runtime_error>([&] { HipHostTensor::from_bytes(SAMHIP_TYPE_Q8_0, 1, 64, b); },
                                         "non-finite or invalid"));
    }
    // F16: every element is checked; -2 and a subnormal decode exactly
    std::vector<uint8_t> h(64, 0);
    h[0] = 0x00, h[1] = 0xc0;   // -2
    h[2] = 0x01, h[3] = 0x00;   // 2^-24
    const std::vector<float> hf = HipHostTensor::from_bytes(SAMHIP_TYPE_F16, 1, 32, h).as_f32();
    CHECK(hf[0] == -2.f && hf[1] == std::ldexp(1.f, -24) && hf[2] == 0.f);
    h[62] = 0x00, h[63] = 0x7c;   // +inf
    CHECK(throws<std::runtime_error>([&] { HipHostTensor::from_bytes(SAMHIP_TYPE_F16, 1, 32, h); }, "non-finite"));
    // half_to_float agrees with the oracle's conversion on every binary16 value
    bool same = true;
    for (uint32_t b = 0; b < 65536; ++b) {
        const float a = half_to_float(uint16_t(b)), o = or_fp16_to_fp32(uint16_t(b));
        uint32_t x, y;
        std::memcpy(&x, &a, 4);
        std::memcpy(&y, &o, 4);
        same = same && (x == y || (std::isnan(a) && std::isnan(o)));
    }
    CHECK(same);
    // wrong sizes and types
    CHECK(throws<std::runtime_error>([&] { HipHostTensor::from_bytes(SAMHIP_TYPE_Q8_0, 1, 64, blk); }, "layout"));
    CHECK(throws<std::runtime_error>([&] { HipHostTensor::from_bytes(SAMHIP_TYPE_Q4_K, 1, 256, {}); }, "type"));
    CHECK(feature_cache_level_type(2, SAMHIP_TYPE_Q8_0) == SAMHIP_TYPE_F32);
    CHECK(feature_cache_level_type(1, SAMHIP_TYPE_Q8_0) == SAMHIP_TYPE_Q8_0);
    CHECK(feature_cache_level_type(2, SAMHIP_TYPE_F16) == SAMHIP_TYPE_F16);
}

// ---------------------------------------------------------------------------

double max_row_rel_l2(const std::vector<float>& y, const std::vector<float>& ref, int m, int n) {
    double worst = 0;
    for (int i = 0; i < m; ++i) {
        double num = 0, den = 0;
        for (int j = 0; j < n; ++j) {
            const double d = double(y[size_t(i) * n + j]) - ref[size_t(i) * n + j];
            num += d * d;
            den += double(ref[size_t(i) * n + j]) * ref[size_t(i) * n + j];
        }
        worst = std::max(worst, std::sqrt(num / (den > 0 ? den : 1e-30)));
    }
    return worst;
}

void test_gpu() {
    using namespace sam;
    HipBackend backend = HipBackend::make(0, HipComputeMode::Q8Native);
    CHECK(backend.device_name().find("gfx950") != std::string::npos);
    CHECK(std::string(backend.arithmetic_profile()) == "ggml-quantized-hip-native-v1");
    CHECK(throws<std::runtime_error>([] { HipBackend::make(1 << 20); }, "out of range"));

    // a text-encoder fc1 (M = 32) and a ViT qkv (M = 300) in Q4_K, and a
    // Q8_0 embedding gather, through one graph
    const int k = 1024, n = 384, m_small = 32, m_tall = 300, vocab = 50;
    std::vector<float> wf(size_t(n) * k), xs(size_t(m_small) * k), xt(size_t(m_tall) * k), emb(size_t(vocab) * k);
    or_rng_normal(0, 0.f, 0.02f, wf.data(), int64_t(wf.size()));
    or_rng_normal(1, 0.f, 1.f, xs.data(), int64_t(xs.size()));
    or_rng_normal(2, 0.f, 1.f, xt.data(), int64_t(xt.size()));
    or_rng_normal(3, 0.f, 1.f, emb.data(), int64_t(emb.size()));
    const size_t wrow = size_t(or_row_bytes(OR_Q4_K, k)), erow = size_t(or_row_bytes(OR_Q8_0, k));
    std::vector<uint8_t> wq(wrow * n), eq(erow * vocab);
    or_quantize_chunk(OR_Q4_K, wf.data(), wq.data(), n, k);
    or_quantize_chunk(OR_Q8_0, emb.data(), eq.data(), vocab, k);
    check_status(samhip_validate_quantized_payload(SAMHIP_TYPE_Q4_K, k, n, wq.data(), wq.size()));

    void* d_w = backend.alloc(wq.size());
    void* d_e = backend.alloc(eq.size());
    void* d_xs = backend.alloc(xs.size() * 4);
    void* d_xt = backend.alloc(xt.size() * 4);
    void* d_ys = backend.alloc(size_t(m_small) * n * 4);
    void* d_yt = backend.alloc(size_t(m_tall) * n * 4);
    const std::vector<int32_t> ids{7, 0, 49, 7};
    void* d_ids = backend.alloc(ids.size() * 4);
    void* d_rows = backend.alloc(ids.size() * k * 4);
    backend.upload(d_w, wq.data(), wq.size());
    backend.upload(d_e, eq.data(), eq.size());
    backend.upload(d_xs, xs.data(), xs.size() * 4);
    backend.upload(d_xt, xt.data(), xt.size() * 4);
    backend.upload(d_ids, ids.data(), ids.size() * 4);

    const samhip_tensor w = make_tensor(SAMHIP_TYPE_Q4_K, k, n, 144, wrow, d_w);
    HipGraphExecution graph(&backend);
    graph.add({HipOp::MulMat, "text.fc1", {"w", "xs"}, {w, make_tensor(SAMHIP_TYPE_F32, k, m_small, 4, 4 * k, d_xs)},
               make_tensor(SAMHIP_TYPE_F32, n, m_small, 4, 4 * n, d_ys)});
    graph.add({HipOp::MulMat, "vit.qkv", {"w", "xt"}, {w, make_tensor(SAMHIP_TYPE_F32, k, m_tall, 4, 4 * k, d_xt)},
               make_tensor(SAMHIP_TYPE_F32, n, m_tall, 4, 4 * n, d_yt)});
    graph.add({HipOp::GetRows, "text.embed", {"token_embd", "ids"},
               {make_tensor(SAMHIP_TYPE_Q8_0, k, vocab, 34, erow, d_e),
                make_tensor(SAMHIP_TYPE_I32, int64_t(ids.size()), 1, 4, 4 * ids.size(), d_ids)},
               make_tensor(SAMHIP_TYPE_F32, k, int64_t(ids.size()), 4, 4 * k, d_rows)});
    HipRuntimeStats stats;
    graph.compute(stats);
    CHECK(stats.hip_nodes == 3 && stats.activation_requests == 2);
    CHECK(stats.activation_allocation_peak_bytes > 0);

    std::vector<float> ys(size_t(m_small) * n), yt(size_t(m_tall) * n), rows(ids.size() * k);
    backend.download(ys.data(), d_ys, ys.size() * 4);
    backend.download(yt.data(), d_yt, yt.size() * 4);
    backend.download(rows.data(), d_rows, rows.size() * 4);
    std::vector<float> rs(ys.size()), rt(yt.size()), decoded(emb.size());
    or_mul_mat_native(OR_Q4_K, wq.data(), int64_t(wrow), xs.data(), k, rs.data(), n, m_small, k, OR_Q8_ROUND_X86, 0);
    or_mul_mat_native(OR_Q4_K, wq.data(), int64_t(wrow), xt.data(), k, rt.data(), n, m_tall, k, OR_Q8_ROUND_X86, 0);
    or_dequantize(OR_Q8_0, eq.data(), decoded.data(), vocab, k);
    const double e1 = max_row_rel_l2(ys, rs, m_small, n), e2 = max_row_rel_l2(yt, rt, m_tall, n);
    std::printf("gpu: text.fc1 max row rel L2 %.3g, vit.qkv %.3g\n", e1, e2);
    CHECK(e1 <= 1e-3 && e2 <= 1e-3);
    bool rows_ok = true;
    for (size_t i = 0; i < ids.size(); ++i)
        rows_ok = rows_ok && std::memcmp(&rows[i * k], &decoded[size_t(ids[i]) * k], size_t(k) * 4) == 0;
    CHECK(rows_ok);

    // an unsupported node stops the graph before any kernel runs
    std::vector<float> sentinel(ys.size(), 7.f);
    backend.upload(d_ys, sentinel.data(), sentinel.size() * 4);
    HipGraphExecution bad(&backend);
    bad.add({HipOp::MulMat, "ok", {"w", "xs"}, {w, make_tensor(SAMHIP_TYPE_F32, k, m_small, 4, 4 * k, d_xs)},
             make_tensor(SAMHIP_TYPE_F32, n, m_small, 4, 4 * n, d_ys)});
    bad.add({HipOp::MulMat, "bad", {"w", "xs"}, {w, make_tensor(SAMHIP_TYPE_F16, k, m_small, 2, 2 * k, d_xs)},
             make_tensor(SAMHIP_TYPE_F32, n, m_small, 4, 4 * n, d_ys)});
    HipRuntimeStats s2;
    CHECK(throws<std::runtime_error>([&] { bad.compute(s2); }, "MUL_MAT tensor bad"));
    backend.download(ys.data(), d_ys, ys.size() * 4);
    CHECK(s2.hip_nodes == 0 && ys == sentinel);
    // bad shapes surface as std::invalid_argument from the operator itself
    CHECK(throws<std::invalid_argument>([&] {
        backend.mul_mat(w, make_tensor(SAMHIP_TYPE_F32, k - 256, m_small, 4, 4 * k, d_xs),
                        make_tensor(SAMHIP_TYPE_F32, n, m_small, 4, 4 * n, d_ys));
    }, "activation width"));

    for (void* p : {d_w, d_e, d_xs, d_xt, d_ys, d_yt, d_ids, d_rows}) backend.free(p);

    // feature caches of a neck-level map (144 x 144 x 256): device cast,
    // host snapshot, re-upload with device decode
    const int64_t fr = 144 * 144, fc = 256;
    std::vector<float> feat(size_t(fr * fc));
    or_rng_normal(9, 0.f, 2.f, feat.data(), int64_t(feat.size()));
    feat[5] = 1e6f;   // beyond F16 range in a row that Q8_0 still represents
    void* d_feat = backend.alloc(feat.size() * 4);
    void* d_back = backend.alloc(feat.size() * 4);
    backend.upload(d_feat, feat.data(), feat.size() * 4);
    // Q8_0: bytes equal the oracle's x86 quantizer, decode equals to_float
    const HipHostTensor q8 = HipHostTensor::capture(backend, static_cast<float*>(d_feat), fr, fc, SAMHIP_TYPE_Q8_0);
    std::vector<uint8_t> ref_q(q8.size_bytes());
    or_quantize_q8_0(feat.data(), ref_q.data(), fr, fc, OR_Q8_ROUND_X86);
    CHECK(q8.bytes() == ref_q);
    std::vector<float> ref_f(feat.size());
    or_dequantize(OR_Q8_0, ref_q.data(), ref_f.data(), fr, fc);
    CHECK(q8.as_f32() == ref_f);
    q8.upload_f32(backend, static_cast<float*>(d_back));
    std::vector<float> back(feat.size());
    backend.download(back.data(), d_back, back.size() * 4);
    CHECK(back == ref_f);
    q8.validate_shape(fc, 144, 144, 1);
    // F16: round to nearest even per value; the 1e6 overflows and is rejected
    CHECK(throws<std::runtime_error>([&] {
        HipHostTensor::capture(backend, static_cast<float*>(d_feat), fr, fc, SAMHIP_TYPE_F16);
    }, "non-finite"));
    feat[5] = 3.f;
    backend.upload(d_feat, feat.data(), feat.size() * 4);
    const HipHostTensor f16 = HipHostTensor::capture(backend, static_cast<float*>(d_feat), fr, fc, SAMHIP_TYPE_F16);
    std::vector<uint16_t> ref_h(feat.size());
    or_fp32_to_fp16_rows(feat.data(), ref_h.data(), int64_t(feat.size()));
    CHECK(std::memcmp(f16.bytes().data(), ref_h.data(), f16.size_bytes()) == 0);
    f16.upload_f32(backend, static_cast<float*>(d_back));
    backend.download(back.data(), d_back, back.size() * 4);
    CHECK(back == f16.as_f32());
    backend.free(d_feat);
    backend.free(d_back);
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "--cpu";
    try {
        if (mode == "--cpu") {
            test_options();
            test_flags();
            test_policy();
            test_status_mapping_without_device();
            test_no_device();
            test_feature_cache_cpu();
        } else if (mode == "--gpu") {
            test_gpu();
        } else {
            std::fprintf(stderr, "usage: test_host --cpu | --gpu\n");
            return 2;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "unexpected exception: %s\n", e.what());
        return 1;
    }
    std::printf("%s: %d checks, %d failed\n", mode.c_str(), g_checks, g_failures);
    return g_failures ? 1 : 0;
}
