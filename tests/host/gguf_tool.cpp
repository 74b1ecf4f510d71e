// Test driver of the GGUF reader and weight upload
// (sam.cpp_amd/host/gguf_reader.hpp), run by tests/test_gguf.py:
//   gguf_tool inspect  <file>      parse; print the tensor table and metadata as JSON
//   gguf_tool contract <file>      the typed-getter checks of the reference's
//                                  loader test on its probe fixture
//                                  (tests/api/test_contracts.cpp:369-385)
//   gguf_tool profile  <file>      resolve the storage profile, check every
//                                  tensor's type against it and validate the
//                                  quantized payloads (no device)
//   gguf_tool gpu      <file> <M>  load the quantized tensors onto device 0,
//                                  check the device bytes equal the file's and
//                                  run each as Y = X W^T with M random rows,
//                                  against the oracle's native product
//   gguf_tool vision-params <file> [relaxed]
//                                  the encoder hyperparameters as JSON, read
//                                  strictly (the reference's fixed SAM 3
//                                  values) or relaxed (any structure)
//   gguf_tool encode   <file> <image.f32> <out prefix> [f32|f16]
//                                  load vit.* / neck.det.* onto device 0, run
//                                  the image encoder (sam.cpp_amd/host/
//                                  vision_encoder.hpp) on the raw F32 planes
//                                  and write the ViT output <prefix>.features.f32
//                                  and <prefix>.level<i>.f32 per neck level
// A rejected file prints {"error": "<message>"} and exits with status 3.
#include "gguf_reader.hpp"
#include "ggml_oracle.h"
#include "vision_encoder.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

std::string json_string(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') {
            o += '\\';
            o += char(c);
        } else if (c < 0x20 || c >= 0x7f) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", c);
            o += buf;
        } else {
            o += char(c);
        }
    }
    return o + "\"";
}

int inspect(const std::string& path) {
    sam::GgufReader r(path);
    std::printf("{\"size\": %llu, \"data_offset\": %llu, \"tensors\": [", (unsigned long long)r.size(),
                (unsigned long long)r.data_offset());
    for (size_t i = 0; i < r.tensors().size(); ++i) {
        const auto& t = r.tensors()[i];
        std::printf("%s{\"name\": %s, \"dims\": [", i ? ", " : "", json_string(t.name).c_str());
        for (size_t d = 0; d < t.dims.size(); ++d) std::printf("%s%lld", d ? ", " : "", (long long)t.dims[d]);
        std::printf("], \"ne\": [%lld, %lld, %lld, %lld], \"type\": %d, \"offset\": %llu, \"size\": %llu}",
                    (long long)t.ne[0], (long long)t.ne[1], (long long)t.ne[2], (long long)t.ne[3], t.type,
                    (unsigned long long)t.offset, (unsigned long long)t.size_bytes);
    }
    std::printf("]}\n");
    return 0;
}

int contract(const std::string& path) {
    using sam::GgufType;
    sam::GgufReader r(path);
    int failures = 0;
    auto check = [&](bool ok, const char* what) {
        if (!ok) {
            ++failures;
            std::printf("FAIL %s\n", what);
        }
    };
    auto rejects = [&](const std::function<void()>& f, const char* what) {
        bool thrown = false;
        try {
            f();
        } catch (const std::runtime_error&) {
            thrown = true;
        }
        check(thrown, what);
    };
    check(r.u32("probe.scalar") == 17 && r.string("probe.label") == "labelx", "typed metadata");
    const auto& indices = r.array("probe.indices", GgufType::U32, 2);
    check(indices.elements == std::vector<uint64_t>{3, 5}, "typed array");
    const auto& labels = r.array("probe.labels", GgufType::String, 2);
    check(labels.strings.at(1) == "second", "string array");
    check(r.tensors().size() == 1 && r.tensors()[0].dims == std::vector<int64_t>{1, 3, 2},
          "leading singleton or tensor dimensions");
    float payload[6] = {};
    r.read(r.tensors()[0].offset, payload, sizeof payload);
    const float want[6] = {-2, -1, 0, 1, 2, 3};
    check(std::memcmp(payload, want, sizeof want) == 0, "tensor payload");
    rejects([&] { r.u32("general.architecture"); }, "wrong scalar type reached a typed getter");
    rejects([&] { r.array("probe.scalar", GgufType::U32, 1); }, "scalar reached an array getter");
    rejects([&] { r.array("probe.labels", GgufType::U32, 2); }, "wrong array element type was accepted");
    rejects([&] { r.array("probe.indices", GgufType::U32, 3); }, "wrong array count was accepted");
    rejects([&] { r.string("missing.key"); }, "missing key was accepted");
    std::printf("contract: %d failed\n", failures);
    return failures ? 1 : 0;
}

int profile(const std::string& path) {
    sam::GgufReader r(path);
    const auto expected = sam::expected_tensor_types(r);
    int constrained = 0;
    for (const auto& t : r.tensors()) {
        const int32_t want = expected(t);
        if (want < 0) continue;
        ++constrained;
        if (want != t.type)
            throw std::runtime_error("incompatible SAM 3 tensor precision: " + t.name + " is " + sam::type_name(t.type) +
                                     ", its storage profile requires " + sam::type_name(want));
    }
    for (const auto& t : r.tensors()) sam::validate_tensor_payload(t, r.tensor_bytes(t));
    std::printf("{\"ok\": true, \"constrained\": %d}\n", constrained);
    return 0;
}

double max_row_rel_l2(const std::vector<float>& y, const std::vector<float>& ref, int64_t m, int64_t n) {
    double worst = 0;
    for (int64_t i = 0; i < m; ++i) {
        double num = 0, den = 0;
        for (int64_t j = 0; j < n; ++j) {
            const double d = double(y[size_t(i * n + j)]) - ref[size_t(i * n + j)];
            num += d * d;
            den += double(ref[size_t(i * n + j)]) * ref[size_t(i * n + j)];
        }
        worst = std::max(worst, std::sqrt(num / (den > 0 ? den : 1e-30)));
    }
    return worst;
}

int gpu(const std::string& path, int64_t m) {
    sam::GgufReader r(path);
    sam::HipBackend backend = sam::HipBackend::make(0, sam::HipComputeMode::Q8Native);
    sam::DeviceWeights weights(backend);
    weights.load(r, [](const sam::GgufTensorInfo& t) { return sam::is_quantized_linear_type(t.type); },
                 sam::expected_tensor_types(r));
    std::printf("{\"loaded\": %zu, \"bytes\": %llu, \"products\": [", weights.count(),
                (unsigned long long)weights.bytes());
    bool first = true;
    uint64_t seed = 11;
    for (const auto& info : r.tensors()) {
        if (!weights.has(info.name)) continue;
        const sam::DeviceTensor& w = weights[info.name];
        const int64_t k = info.ne[0], n = info.ne[1];
        // the device holds the file's bytes unchanged
        std::vector<uint8_t> file = r.tensor_bytes(info), dev(file.size());
        backend.download(dev.data(), w.data, dev.size());
        const bool same = dev == file;
        std::vector<float> x(size_t(m * k)), y(size_t(m * n)), ref(y.size());
        or_rng_normal(seed++, 0.f, 1.f, x.data(), int64_t(x.size()));
        void* dx = backend.alloc(x.size() * 4);
        void* dy = backend.alloc(y.size() * 4);
        backend.upload(dx, x.data(), x.size() * 4);
        backend.mul_mat(w.view(), sam::make_tensor(SAMHIP_TYPE_F32, k, m, 4, size_t(4 * k), dx),
                        sam::make_tensor(SAMHIP_TYPE_F32, n, m, 4, size_t(4 * n), dy));
        backend.download(y.data(), dy, y.size() * 4);
        backend.free(dx);
        backend.free(dy);
        or_mul_mat_native(info.type, file.data(), size_t(w.view().nb[1]), x.data(), size_t(k), ref.data(), n, m, k,
                          OR_Q8_ROUND_X86, 0);
        std::printf("%s{\"name\": %s, \"type\": %d, \"k\": %lld, \"n\": %lld, \"bytes_equal\": %s, "
                    "\"max_row_rel_l2\": %.6g}",
                    first ? "" : ", ", json_string(info.name).c_str(), info.type, (long long)k, (long long)n,
                    same ? "true" : "false", max_row_rel_l2(y, ref, m, n));
        std::fflush(stdout);
        first = false;
    }
    std::printf("]}\n");
    return 0;
}

int vision_params(const std::string& path, bool relaxed) {
    sam::GgufReader r(path);
    const sam::VisionParameters p = relaxed ? sam::VisionParameters::read_relaxed(r) : sam::VisionParameters::read(r);
    std::printf("{\"image_size\": %d, \"patch\": %d, \"embed\": %d, \"blocks\": %d, \"heads\": %d, \"mlp\": %d, "
                "\"window\": %d, \"neck_dim\": %d, \"global_blocks\": [",
                p.image_size, p.patch, p.embed, p.blocks, p.heads, p.mlp, p.window, p.neck_dim);
    for (size_t i = 0; i < p.global_blocks.size(); ++i) std::printf("%s%d", i ? ", " : "", p.global_blocks[i]);
    std::printf("]}\n");
    return 0;
}

// The reduced test checkpoints are read relaxed; a full SAM 3 file passes
// the strict read too.
int encode(const std::string& path, const std::string& image_path, const std::string& prefix, bool f16) {
    sam::GgufReader r(path);
    const sam::VisionParameters p = sam::VisionParameters::read_relaxed(r);
    sam::HipBackend backend = sam::HipBackend::make(0, sam::HipComputeMode::Q8Native);
    sam::DeviceWeights weights(backend);
    weights.load(r, [](const sam::GgufTensorInfo& t) {
        return t.name.rfind("vit.", 0) == 0 || t.name.rfind("neck.det.", 0) == 0;
    });
    sam::HipVisionEncoder encoder(backend, weights, p, f16 ? SAMHIP_TYPE_F16 : SAMHIP_TYPE_F32);
    const size_t image_floats = size_t(3) * p.image_size * p.image_size;
    std::vector<float> image(image_floats);
    FILE* f = std::fopen(image_path.c_str(), "rb");
    if (!f || std::fread(image.data(), 4, image_floats, f) != image_floats) {
        if (f) std::fclose(f);
        throw std::runtime_error("cannot read the image planes");
    }
    std::fclose(f);
    void* dimage = backend.alloc(image_floats * 4);
    backend.upload(dimage, image.data(), image_floats * 4);
    const bool level3 = weights.has("neck.det.3.conv_1x1.weight");
    float* levels[4] = {nullptr, nullptr, nullptr, nullptr};
    for (int i = 0; i < (level3 ? 4 : 3); ++i) {
        const size_t side = size_t(encoder.level_side(i));
        levels[i] = static_cast<float*>(backend.alloc(side * side * size_t(p.neck_dim) * 4));
    }
    encoder.encode(static_cast<const float*>(dimage), levels);
    backend.synchronize();
    {
        const size_t n = size_t(p.grid()) * p.grid() * size_t(p.embed);
        std::vector<float> x(n);
        backend.download(x.data(), encoder.features(), n * 4);
        const std::string name = prefix + ".features.f32";
        FILE* o = std::fopen(name.c_str(), "wb");
        if (!o || std::fwrite(x.data(), 4, n, o) != n) {
            if (o) std::fclose(o);
            throw std::runtime_error("cannot write " + name);
        }
        std::fclose(o);
    }
    std::printf("{\"loaded\": %zu, \"grid\": %d, \"dim\": %d, \"levels\": [", weights.count(), p.grid(),
                p.neck_dim);
    for (int i = 0; i < 4 && levels[i]; ++i) {
        const size_t side = size_t(encoder.level_side(i)), n = side * side * size_t(p.neck_dim);
        std::vector<float> out(n);
        backend.download(out.data(), levels[i], n * 4);
        const std::string name = prefix + ".level" + std::to_string(i) + ".f32";
        FILE* o = std::fopen(name.c_str(), "wb");
        if (!o || std::fwrite(out.data(), 4, n, o) != n) {
            if (o) std::fclose(o);
            throw std::runtime_error("cannot write " + name);
        }
        std::fclose(o);
        std::printf("%s%zu", i ? ", " : "", side);
        backend.free(levels[i]);
    }
    std::printf("]}\n");
    backend.free(dimage);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: gguf_tool inspect|contract|profile <file> | gpu <file> <M> | "
                             "vision-params <file> [relaxed] | encode <file> <image.f32> <out prefix> [f32|f16]\n");
        return 2;
    }
    const std::string mode = argv[1], path = argv[2];
    try {
        if (mode == "inspect") return inspect(path);
        if (mode == "contract") return contract(path);
        if (mode == "profile") return profile(path);
        if (mode == "gpu" && argc > 3) return gpu(path, std::atoll(argv[3]));
        if (mode == "vision-params") return vision_params(path, argc > 3 && std::string(argv[3]) == "relaxed");
        if (mode == "encode" && argc > 4)
            return encode(path, argv[3], argv[4], argc > 5 && std::string(argv[5]) == "f16");
        std::fprintf(stderr, "unknown mode %s\n", mode.c_str());
        return 2;
    } catch (const std::exception& e) {
        std::printf("{\"error\": %s}\n", json_string(e.what()).c_str());
        return 3;
    }
}
