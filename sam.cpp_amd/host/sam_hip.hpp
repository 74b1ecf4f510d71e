// C++17 host layer over the samhip C ABI: the pieces SAM.cpp's runtime needs
// to select an MI355X backend and run its quantized linears through it.
//
//  * Backend / BackendOptions with the HIP fields and their validation
//    (mirrors sam::Backend and validate_backend_options:
//    include/sam/types.hpp:12-24, src/common/input_validation.hpp:20-44);
//  * the --backend / --hip-device / --hip-compute command-line options
//    (support/image_io/image_support.hpp:95-130);
//  * HipBackend: RAII owner of one samhip context, the make_*_backend driver
//    factory (src/runtime/ggml/backends/cuda.hpp:156-189), mapping the C
//    status codes to std::invalid_argument / std::runtime_error as the
//    reference does (src/runtime/ggml/workspace.hpp:174-177);
//  * HipGraphExecution: the prepare / compute split of GraphExecution
//    (src/runtime/ggml/graph.hpp:56-100): every node's support is checked
//    before anything runs, compute counts device nodes (hip_nodes);
//  * the image quantization format policy that decides each linear's GGUF
//    type (src/models/sam3/weights.hpp:48-162, 169-243).
//
// Header-only; link libsamhip.so.
#pragma once

#include "samhip.h"

#include <algorithm>
#include <array>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace sam {

enum class Backend { Auto, Cpu, Metal, Cuda, Hip };
enum class CudaComputeMode { F32, F16 };
enum class CpuComputeMode { F32, NativeQuantized };
// Q8Native: activations packed to the weight's ggml vec_dot_type per call;
// F16: activations rounded to fp16.  Weights are fp16(to_float(W)) in both.
enum class HipComputeMode { Q8Native, F16 };

struct BackendOptions {
    Backend backend = Backend::Auto;
    int threads = 4;
    int cuda_device = 0;
    CudaComputeMode cuda_compute = CudaComputeMode::F32;
    CpuComputeMode cpu_compute = CpuComputeMode::F32;
    int hip_device = 0;                                 // index among visible HIP devices
    HipComputeMode hip_compute = HipComputeMode::Q8Native;
};

// Device-side counters reported by the HIP backend (the HIP analogues of
// RuntimeStats::cuda_nodes and the activation_* fields, include/sam/types.hpp:45-58).
struct HipRuntimeStats {
    std::uint64_t hip_nodes = 0;
    std::uint64_t activation_requests = 0;
    std::uint64_t activation_payload_peak_bytes = 0, activation_allocation_peak_bytes = 0;
};

inline void validate_backend_options(const BackendOptions& o) {
    if (o.backend != Backend::Auto && o.backend != Backend::Cpu && o.backend != Backend::Metal &&
        o.backend != Backend::Cuda && o.backend != Backend::Hip)
        throw std::invalid_argument("unknown SAM backend");
    if (o.threads <= 0) throw std::invalid_argument("CPU thread count must be positive");
    if (o.cuda_device < 0 || (o.backend != Backend::Cuda && o.cuda_device != 0))
        throw std::invalid_argument("CUDA device must be nonnegative and requires an explicit CUDA backend");
    if (o.cuda_compute != CudaComputeMode::F32 && o.cuda_compute != CudaComputeMode::F16)
        throw std::invalid_argument("unknown CUDA compute mode");
    if (o.cuda_compute != CudaComputeMode::F32 && o.backend != Backend::Cuda)
        throw std::invalid_argument("reduced CUDA compute requires an explicit CUDA backend");
    if (o.cpu_compute != CpuComputeMode::F32 && o.cpu_compute != CpuComputeMode::NativeQuantized)
        throw std::invalid_argument("unknown CPU compute mode");
    if (o.cpu_compute != CpuComputeMode::F32 && o.backend != Backend::Cpu)
        throw std::invalid_argument("native quantized CPU compute requires an explicit CPU backend");
    if (o.hip_device < 0 || (o.backend != Backend::Hip && o.hip_device != 0))
        throw std::invalid_argument("HIP device must be nonnegative and requires an explicit HIP backend");
    if (o.hip_compute != HipComputeMode::Q8Native && o.hip_compute != HipComputeMode::F16)
        throw std::invalid_argument("unknown HIP compute mode");
    if (o.hip_compute != HipComputeMode::Q8Native && o.backend != Backend::Hip)
        throw std::invalid_argument("HIP compute mode requires an explicit HIP backend");
}

// One "--name value" pair of the backend options; returns false for names it
// does not own.  finish_backend_flags() applies the cross-option rules once
// all flags are read.
inline bool parse_backend_flag(const std::string& name, const std::string& value, BackendOptions& o,
                               std::vector<std::string>& seen) {
    auto nonnegative = [&](const std::string& v) {
        if (v.empty() || v.find_first_not_of("0123456789") != std::string::npos)
            throw std::invalid_argument(name + " must be a nonnegative integer");
        errno = 0;
        const long x = std::strtol(v.c_str(), nullptr, 10);
        if (errno == ERANGE || x > 1 << 20) throw std::invalid_argument(name + " is out of range");
        return int(x);
    };
    if (name == "--backend") {
        if (value == "auto") o.backend = Backend::Auto;
        else if (value == "cpu") o.backend = Backend::Cpu;
        else if (value == "metal") o.backend = Backend::Metal;
        else if (value == "cuda") o.backend = Backend::Cuda;
        else if (value == "hip") o.backend = Backend::Hip;
        else throw std::invalid_argument("--backend must be auto, cpu, metal, cuda, or hip");
    } else if (name == "--hip-device") {
        o.hip_device = nonnegative(value);
    } else if (name == "--hip-compute") {
        if (value == "q8-native") o.hip_compute = HipComputeMode::Q8Native;
        else if (value == "f16") o.hip_compute = HipComputeMode::F16;
        else throw std::invalid_argument("--hip-compute must be q8-native or f16");
    } else {
        return false;
    }
    seen.push_back(name);
    return true;
}

inline void finish_backend_flags(const BackendOptions& o, const std::vector<std::string>& seen) {
    auto given = [&](const char* n) { return std::find(seen.begin(), seen.end(), n) != seen.end(); };
    if (given("--hip-device") && o.backend != Backend::Hip)
        throw std::invalid_argument("--hip-device requires --backend hip");
    if (given("--hip-compute") && o.backend != Backend::Hip)
        throw std::invalid_argument("--hip-compute requires --backend hip");
    validate_backend_options(o);
}

inline const char* backend_name(Backend b) {
    switch (b) {
        case Backend::Auto: return "auto";
        case Backend::Cpu: return "cpu";
        case Backend::Metal: return "metal";
        case Backend::Cuda: return "cuda";
        case Backend::Hip: return "hip";
    }
    return "unknown";
}

// ---------------------------------------------------------------------------
// C ABI status -> the reference's exception types
// ---------------------------------------------------------------------------

inline std::string samhip_message() {
    std::string msg(samhip_last_error(nullptr, 0) + 1, '\0');
    samhip_last_error(&msg[0], msg.size());
    msg.resize(msg.size() - 1);
    return msg;
}

inline void check_status(int status) {
    if (status == SAMHIP_OK) return;
    if (status == SAMHIP_ERR_INVALID_ARGUMENT) throw std::invalid_argument(samhip_message());
    throw std::runtime_error(samhip_message());
}

// ggml tensor view in the C ABI's terms (ne = elements, nb = byte strides).
inline samhip_tensor make_tensor(int32_t type, int64_t ne0, int64_t ne1, std::size_t nb0, std::size_t nb1, void* data) {
    samhip_tensor t{};
    t.type = type;
    t.ne[0] = ne0;
    t.ne[1] = ne1;
    t.ne[2] = t.ne[3] = 1;
    t.nb[0] = nb0;
    t.nb[1] = nb1;
    t.nb[2] = t.nb[3] = nb1 * std::size_t(ne1);
    t.data = data;
    return t;
}

inline const char* type_name(int32_t type) {
    switch (type) {
        case SAMHIP_TYPE_F32: return "f32";
        case SAMHIP_TYPE_F16: return "f16";
        case SAMHIP_TYPE_Q8_0: return "q8_0";
        case SAMHIP_TYPE_Q4_K: return "q4_K";
        case SAMHIP_TYPE_Q5_K: return "q5_K";
        case SAMHIP_TYPE_Q6_K: return "q6_K";
        case SAMHIP_TYPE_Q8_K: return "q8_K";
        case SAMHIP_TYPE_I32: return "i32";
        default: return "?";
    }
}

// ---------------------------------------------------------------------------
// Backend driver
// ---------------------------------------------------------------------------

class HipBackend {
public:
    // make_hip_backend: device index among visible HIP devices.
    static HipBackend make(int device, HipComputeMode compute = HipComputeMode::Q8Native) {
        int count = 0;
        check_status(samhip_device_count(&count));
        if (count == 0) throw std::runtime_error("requested HIP backend has no visible devices");
        if (device < 0 || device >= count)
            throw std::runtime_error("requested HIP device index is out of range for visible devices");
        samhip_options o{SAMHIP_ABI_VERSION, device,
                         compute == HipComputeMode::F16 ? SAMHIP_COMPUTE_F16 : SAMHIP_COMPUTE_Q8_NATIVE,
                         SAMHIP_Q8_ROUND_X86};
        samhip_context* ctx = nullptr;
        check_status(samhip_context_create(&o, &ctx));
        return HipBackend(ctx, device, compute);
    }
    HipBackend(HipBackend&& other) noexcept { *this = std::move(other); }
    HipBackend& operator=(HipBackend&& other) noexcept {
        if (this != &other) {
            reset();
            ctx_ = std::exchange(other.ctx_, nullptr);
            device_ = other.device_;
            compute_ = other.compute_;
        }
        return *this;
    }
    HipBackend(const HipBackend&) = delete;
    HipBackend& operator=(const HipBackend&) = delete;
    ~HipBackend() { reset(); }

    samhip_context* handle() const { return ctx_; }
    int device() const { return device_; }
    HipComputeMode compute() const { return compute_; }

    std::string device_name() const { return query().device_name; }
    // Runtime arithmetic contract, next to the reference's profile strings
    // (src/runtime/ggml/runtime.hpp:99-107).
    const char* arithmetic_profile() const {
        return compute_ == HipComputeMode::F16 ? "ggml-quantized-hip-f16-v1" : "ggml-quantized-hip-native-v1";
    }

    samhip_exec_info query() const {
        samhip_exec_info info{};
        check_status(samhip_query(ctx_, &info));
        return info;
    }

    void* alloc(std::size_t bytes) {
        void* p = nullptr;
        check_status(samhip_buffer_alloc(ctx_, bytes, &p));
        return p;
    }
    void free(void* p) { check_status(samhip_buffer_free(ctx_, p)); }
    void upload(void* dst, const void* src, std::size_t bytes) { check_status(samhip_tensor_set(ctx_, dst, src, bytes)); }
    void download(void* dst, const void* src, std::size_t bytes) { check_status(samhip_tensor_get(ctx_, dst, src, bytes)); }
    void synchronize() { check_status(samhip_synchronize(ctx_)); }

    static bool supports_mul_mat(const samhip_tensor& w, const samhip_tensor& x, const samhip_tensor& y) {
        return samhip_supports_mul_mat(&w, &x, &y) != 0;
    }
    void mul_mat(const samhip_tensor& w, const samhip_tensor& x, const samhip_tensor& y) {
        check_status(samhip_mul_mat(ctx_, &w, &x, &y));
    }
    void get_rows(const samhip_tensor& src, const samhip_tensor& ids, const samhip_tensor& dst) {
        check_status(samhip_get_rows(ctx_, &src, &ids, &dst));
    }

private:
    HipBackend(samhip_context* ctx, int device, HipComputeMode compute) : ctx_(ctx), device_(device), compute_(compute) {}
    void reset() {
        if (ctx_) samhip_context_destroy(ctx_);
        ctx_ = nullptr;
    }
    samhip_context* ctx_ = nullptr;
    int device_ = -1;
    HipComputeMode compute_ = HipComputeMode::Q8Native;
};

// ---------------------------------------------------------------------------
// Graph execution over the HIP backend
// ---------------------------------------------------------------------------

enum class HipOp { MulMat, GetRows };

struct HipNode {
    HipOp op;
    std::string name;                 // dst tensor name
    std::string src_names[2];
    samhip_tensor src[2];
    samhip_tensor dst;
};

class HipGraphExecution {
public:
    // `backend` may be null for a graph that is only validated.
    explicit HipGraphExecution(HipBackend* backend) : backend_(backend) {}
    void add(HipNode node) {
        nodes_.push_back(std::move(node));
        validated_ = false;
    }
    // Every node must have a kernel before any runs, so an unsupported
    // operator is a runtime error at the library boundary, not a device fault.
    void prepare() {
        if (validated_) return;
        for (const auto& n : nodes_) {
            bool ok = true;
            if (n.op == HipOp::MulMat) ok = HipBackend::supports_mul_mat(n.src[0], n.src[1], n.dst);
            else ok = get_rows_supported(n);
            if (!ok) {
                std::string message = std::string("no backend supports SAM operation ") +
                                      (n.op == HipOp::MulMat ? "MUL_MAT" : "GET_ROWS") + " tensor " + n.name;
                for (int s = 0; s < 2; ++s)
                    message += " source" + std::to_string(s) + "=" + n.src_names[s] + "/" + type_name(n.src[s].type);
                throw std::runtime_error(message);
            }
        }
        validated_ = true;
    }
    void compute(HipRuntimeStats& stats) {
        prepare();
        if (!backend_) throw std::runtime_error("HIP graph has no backend to run on");
        for (const auto& n : nodes_) {
            if (n.op == HipOp::MulMat) backend_->mul_mat(n.src[0], n.src[1], n.dst);
            else backend_->get_rows(n.src[0], n.src[1], n.dst);
            ++stats.hip_nodes;
            if (n.op == HipOp::MulMat) ++stats.activation_requests;
        }
        const samhip_exec_info info = backend_->query();
        stats.activation_payload_peak_bytes = std::max(stats.activation_payload_peak_bytes, info.activation_payload_peak_bytes);
        stats.activation_allocation_peak_bytes =
            std::max(stats.activation_allocation_peak_bytes, info.activation_allocation_peak_bytes);
    }
    std::size_t size() const { return nodes_.size(); }

private:
    static bool get_rows_supported(const HipNode& n) {
        const int t = n.src[0].type;
        const bool type_ok = t == SAMHIP_TYPE_F32 || t == SAMHIP_TYPE_F16 || t == SAMHIP_TYPE_Q8_0 ||
                             t == SAMHIP_TYPE_Q4_K || t == SAMHIP_TYPE_Q5_K || t == SAMHIP_TYPE_Q6_K;
        return type_ok && n.src[1].type == SAMHIP_TYPE_I32 && n.dst.type == SAMHIP_TYPE_F32 && n.src[0].ne[0] % 32 == 0;
    }
    HipBackend* backend_;
    std::vector<HipNode> nodes_;
    bool validated_ = false;
};

// ---------------------------------------------------------------------------
// Image quantization format policy (which GGUF type each linear is stored in)
// ---------------------------------------------------------------------------

namespace policy {

struct ImageQuantizationProfile {
    const char* name;
    const char* precision;
    int32_t type;
    std::uint32_t file_type;
    bool quantize_text_linear;
};

struct ModularImageQuantizationProfile {
    const char* name;
    const char* precision;
    int32_t type;
    std::uint32_t file_type;
    bool full_preset;
};

inline int32_t block_elems(int32_t type) { return type == SAMHIP_TYPE_Q8_0 ? 32 : 256; }

// Profile tables: names, precisions and GGUF file types must match the
// reference's so that a converted file resolves to the same storage.
inline const ImageQuantizationProfile* image_quantization_profile(const std::string& name) {
    static const std::array<ImageQuantizationProfile, 8> table{{
        {"image-linear-q8_0-v1", "q8_0", SAMHIP_TYPE_Q8_0, 7, true},
        {"image-linear-q6_k-v1", "q6_k", SAMHIP_TYPE_Q6_K, 18, true},
        {"image-linear-q5_k-v1", "q5_k", SAMHIP_TYPE_Q5_K, 16, true},
        {"image-linear-q4_k-v1", "q4_k", SAMHIP_TYPE_Q4_K, 14, true},
        {"image-vision-linear-q8_0-v1", "q8_0", SAMHIP_TYPE_Q8_0, 7, false},
        {"image-vision-linear-q6_k-v1", "q6_k", SAMHIP_TYPE_Q6_K, 18, false},
        {"image-vision-linear-q5_k-v1", "q5_k", SAMHIP_TYPE_Q5_K, 16, false},
        {"image-vision-linear-q4_k-v1", "q4_k", SAMHIP_TYPE_Q4_K, 14, false},
    }};
    for (const auto& p : table)
        if (name == p.name) return &p;
    return nullptr;
}

inline const ModularImageQuantizationProfile* modular_image_quantization_profile(const std::string& name) {
    static const std::array<ModularImageQuantizationProfile, 8> table{{
        {"image-full-linear-q8_0-v1", "q8_0", SAMHIP_TYPE_Q8_0, 7, true},
        {"image-full-linear-q6_k-v1", "q6_k", SAMHIP_TYPE_Q6_K, 18, true},
        {"image-full-linear-q5_k-v1", "q5_k", SAMHIP_TYPE_Q5_K, 16, true},
        {"image-full-linear-q4_k-v1", "q4_k", SAMHIP_TYPE_Q4_K, 14, true},
        {"image-modules-linear-q8_0-v1", "q8_0", SAMHIP_TYPE_Q8_0, 7, false},
        {"image-modules-linear-q6_k-v1", "q6_k", SAMHIP_TYPE_Q6_K, 18, false},
        {"image-modules-linear-q5_k-v1", "q5_k", SAMHIP_TYPE_Q5_K, 16, false},
        {"image-modules-linear-q4_k-v1", "q4_k", SAMHIP_TYPE_Q4_K, 14, false},
    }};
    for (const auto& p : table)
        if (name == p.name) return &p;
    return nullptr;
}

inline const std::array<const char*, 4>& module_order() {
    static const std::array<const char*, 4> order{{"vision", "text", "fusion", "decoder"}};
    return order;
}

// "<prefix><layer>.<suffix>" for some layer in [0, layers) and listed suffix.
inline bool indexed_layer_weight(const std::string& name, const std::string& prefix, int layers,
                                 std::initializer_list<const char*> suffixes) {
    if (name.compare(0, prefix.size(), prefix) != 0) return false;
    std::size_t i = prefix.size(), j = i;
    while (j < name.size() && name[j] >= '0' && name[j] <= '9') ++j;
    if (j == i || j - i > 3 || j >= name.size() || name[j] != '.') return false;
    if (j - i > 1 && name[i] == '0') return false;   // no leading zeros
    const int layer = std::atoi(name.substr(i, j - i).c_str());
    if (layer >= layers) return false;
    const std::string rest = name.substr(j + 1);
    for (const char* s : suffixes)
        if (rest == s) return true;
    return false;
}

inline bool is_image_quantized_linear_weight(const std::string& name, bool quantize_text_linear) {
    if (indexed_layer_weight(name, "vit.blocks.", 32,
                             {"attn.qkv.weight", "attn.proj.weight", "mlp.lin1.weight", "mlp.lin2.weight"}))
        return true;
    return quantize_text_linear &&
           indexed_layer_weight(name, "text.blocks.", 24,
                                {"attn.in_proj.weight", "attn.out_proj.weight", "mlp.fc1.weight", "mlp.fc2.weight"});
}

// The ViT MLP down-projection: 4736-wide rows cannot hold 256-value K-quant
// super-blocks, so K-quant profiles store it as Q8_0.
inline bool is_image_q8_k_fallback_weight(const std::string& name) {
    return indexed_layer_weight(name, "vit.blocks.", 32, {"mlp.lin2.weight"});
}

inline int32_t image_quantized_tensor_type(const std::string& name, const std::vector<int64_t>& dims,
                                           const ImageQuantizationProfile& profile) {
    if (!is_image_quantized_linear_weight(name, profile.quantize_text_linear)) return SAMHIP_TYPE_F32;
    const int32_t block = block_elems(profile.type);
    if (block == 256 && !dims.empty() && dims[0] == 4736 && is_image_q8_k_fallback_weight(name)) return SAMHIP_TYPE_Q8_0;
    if (block == 256 && (dims.empty() || dims[0] % block != 0))
        throw std::runtime_error("K quantization profile has a noncanonical row width: " + name);
    return profile.type;
}

inline bool image_modular_linear_weight(const std::string& name, const std::string& module) {
    if (module == "vision") return is_image_quantized_linear_weight(name, false);
    if (module == "text")
        return name == "text.resizer.weight" ||
               indexed_layer_weight(name, "text.blocks.", 24,
                                    {"attn.in_proj.weight", "attn.out_proj.weight", "mlp.fc1.weight", "mlp.fc2.weight"});
    if (module == "fusion")
        return indexed_layer_weight(name, "fenc.layers.", 6,
                                    {"sa.in_proj_weight", "sa.out_proj.weight", "ca.in_proj_weight",
                                     "ca.out_proj.weight", "linear1.weight", "linear2.weight"});
    if (module != "decoder") return false;
    if (indexed_layer_weight(name, "ddec.layers.", 6,
                             {"sa.in_proj_weight", "sa.out_proj.weight", "ca.in_proj_weight", "ca.out_proj.weight",
                              "ca_text.in_proj_weight", "ca_text.out_proj.weight", "linear1.weight", "linear2.weight"}))
        return true;
    if (indexed_layer_weight(name, "geom.layers.", 3,
                             {"sa.in_proj_weight", "sa.out_proj.weight", "ca.in_proj_weight", "ca.out_proj.weight",
                              "linear1.weight", "linear2.weight"}))
        return true;
    for (const char* head : {"ddec.bbox_embed.layers.", "ddec.presence_token_head.layers.",
                             "seg.mask_predictor.mask_embed.layers."})
        if (indexed_layer_weight(name, head, 3, {"weight"})) return true;
    if (indexed_layer_weight(name, "ddec.ref_point_head.layers.", 2, {"weight"})) return true;
    for (const char* axis : {"x", "y"})
        if (indexed_layer_weight(name, std::string("ddec.boxRPB_embed_") + axis + ".layers.", 2, {"weight"}))
            return true;
    for (const char* fixed : {"scoring.prompt_proj.weight", "scoring.hs_proj.weight",
                              "scoring.prompt_mlp.layers.0.weight", "scoring.prompt_mlp.layers.1.weight",
                              "geom.points_direct_project.weight", "geom.boxes_direct_project.weight",
                              "geom.boxes_pos_enc_project.weight", "geom.points_pool_project.weight",
                              "geom.points_pos_enc_project.weight", "geom.final_proj.weight",
                              "seg.cross_attend_prompt.in_proj_weight", "seg.cross_attend_prompt.out_proj.weight"})
        if (name == fixed) return true;
    return false;
}

inline int32_t image_modular_quantized_tensor_type(const std::string& name, const std::vector<int64_t>& dims,
                                                   const ModularImageQuantizationProfile& profile,
                                                   const std::vector<std::string>& modules) {
    if (dims.size() != 2) return SAMHIP_TYPE_F32;
    bool eligible = false;
    for (const char* m : module_order())
        eligible = eligible || (std::find(modules.begin(), modules.end(), m) != modules.end() &&
                                image_modular_linear_weight(name, m));
    if (!eligible) return SAMHIP_TYPE_F32;
    const int64_t width = dims[0];
    if (width <= 0 || width % 32 != 0) return SAMHIP_TYPE_F32;
    if (profile.type == SAMHIP_TYPE_Q8_0) return profile.type;
    if (width % 256 == 0) return profile.type;
    if (width == 4736 && is_image_q8_k_fallback_weight(name)) return SAMHIP_TYPE_Q8_0;
    return SAMHIP_TYPE_F32;
}

// The accepted lists are exactly the nonempty subsequences of module_order()
// joined by commas (15 of them): the list names each module at most once, in
// that order.  Each candidate is spelled out from a 4-bit mask and compared
// with the whole string.
inline std::vector<std::string> parse_image_quantization_modules(const std::string& csv) {
    if (csv.empty()) throw std::runtime_error("schema-4 quantization module list is empty");
    for (unsigned mask = 1; mask < 16; ++mask) {
        std::vector<std::string> picked;
        std::string spelled;
        for (unsigned i = 0; i < 4; ++i) {
            if (!((mask >> i) & 1u)) continue;
            picked.emplace_back(module_order()[i]);
            spelled += (spelled.empty() ? "" : ",") + picked.back();
        }
        if (spelled == csv) return picked;
    }
    throw std::runtime_error("schema-4 quantization modules must be a nonempty canonical CSV list");
}

}  // namespace policy

}  // namespace sam
