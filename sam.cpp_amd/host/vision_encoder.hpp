// The SAM 3 image encoder over the HIP backend, from a converted
// checkpoint's device tensors: the ViT prefix, its blocks and the detector
// neck, in place of sam3_build_vit_graph + sam3_build_neck_graph
// (src/models/sam3/vision.hpp:278-366) as the image path runs them
// (src/models/sam3/execution.hpp:66-94).  Tensor names and ggml shapes are
// the ones the reference registers (src/models/sam3/tensors.hpp:96-163).
#pragma once

#include "gguf_reader.hpp"

#include <algorithm>
#include <array>
#include <string>
#include <utility>
#include <vector>

namespace sam {

// The encoder hyperparameters of a checkpoint (sam3.vision.* and
// sam3.neck.embedding_length, src/models/sam3/weights.hpp:427-438 and
// 591-600).  read() is strict by default, as the reference loader is: every
// SAM 3 image parameter must hold its fixed value and the global attention
// blocks must be the U32 array {7, 15, 23, 31}.  read_relaxed() accepts any
// encoder of the same structure (the reduced checkpoints of the tests) and
// leaves the shape checks to each tensor.
struct VisionParameters {
    int image_size = 0, patch = 0, embed = 0, blocks = 0, heads = 0, mlp = 0, window = 0, neck_dim = 0;
    std::vector<int> global_blocks;

    int grid() const { return image_size / patch; }
    // the position embedding is stored at a third of the grid and tiled
    // (src/models/sam3/tensors.hpp:99-104)
    int pos_grid() const { return grid() / 3; }
    bool is_global(int block) const {
        return std::find(global_blocks.begin(), global_blocks.end(), block) != global_blocks.end();
    }

    // sam3_image_parameters (src/models/sam3/weights.hpp:427-439)
    static const std::array<std::pair<const char*, uint32_t>, 22>& sam3_values() {
        static const std::array<std::pair<const char*, uint32_t>, 22> v{{
            {"sam3.vision.image_size", 1008}, {"sam3.vision.patch_size", 14},
            {"sam3.vision.embedding_length", 1024}, {"sam3.vision.block_count", 32},
            {"sam3.vision.attention.head_count", 16}, {"sam3.vision.feed_forward_length", 4736},
            {"sam3.vision.window_size", 24}, {"sam3.text.embedding_length", 1024},
            {"sam3.text.attention.head_count", 16}, {"sam3.text.block_count", 24},
            {"sam3.text.context_length", 32}, {"sam3.text.vocab_size", 49408},
            {"sam3.text.output_length", 256}, {"sam3.neck.embedding_length", 256},
            {"sam3.fusion.block_count", 6}, {"sam3.fusion.attention.head_count", 8},
            {"sam3.fusion.feed_forward_length", 2048}, {"sam3.decoder.block_count", 6},
            {"sam3.decoder.attention.head_count", 8}, {"sam3.decoder.feed_forward_length", 2048},
            {"sam3.decoder.query_count", 200}, {"sam3.geometry.block_count", 3}}};
        return v;
    }

    static VisionParameters read(const GgufReader& r) {
        for (const auto& kv : sam3_values())
            if (r.u32(kv.first) != kv.second)
                throw std::runtime_error(std::string("unsupported SAM 3 image parameter: ") + kv.first);
        VisionParameters p = read_relaxed(r);
        const std::vector<int> expected{7, 15, 23, 31};
        if (p.global_blocks != expected) throw std::runtime_error("unsupported SAM 3 global attention block order");
        return p;
    }

    static VisionParameters read_relaxed(const GgufReader& r) {
        VisionParameters p;
        p.image_size = int(r.u32("sam3.vision.image_size"));
        p.patch = int(r.u32("sam3.vision.patch_size"));
        p.embed = int(r.u32("sam3.vision.embedding_length"));
        p.blocks = int(r.u32("sam3.vision.block_count"));
        p.heads = int(r.u32("sam3.vision.attention.head_count"));
        p.mlp = int(r.u32("sam3.vision.feed_forward_length"));
        p.window = int(r.u32("sam3.vision.window_size"));
        p.neck_dim = int(r.u32("sam3.neck.embedding_length"));
        const GgufValue& g = r.value("sam3.vision.global_attention_blocks", GgufType::Array);
        if (g.array_type != GgufType::U32) throw std::runtime_error("incompatible GGUF array: global attention blocks");
        for (uint64_t b : g.elements) p.global_blocks.push_back(int(uint32_t(b)));
        p.validate();
        return p;
    }

    void validate() const {
        if (image_size <= 0 || patch <= 0 || image_size % patch || grid() % 3 || embed <= 0 || heads <= 0 ||
            embed % heads || embed / heads != 64 || blocks <= 0 || mlp <= 0 || window <= 0 || neck_dim <= 0)
            throw std::runtime_error("unsupported SAM 3 image encoder parameters");
        for (size_t i = 0; i < global_blocks.size(); ++i)
            if (global_blocks[i] < 0 || global_blocks[i] >= blocks || (i && global_blocks[i] <= global_blocks[i - 1]))
                throw std::runtime_error("unsupported SAM 3 global attention block order");
    }
};

class HipVisionEncoder {
public:
    // `weights` must hold the vit.* and neck.det.* tensors: F32 norms, biases,
    // embeddings, RoPE tables and neck convolutions; packed Q8_0 / K-quant
    // linears.  They stay owned by `weights`, which must outlive this object.
    // columns_type: the neck's 1x1/3x3 operands (F32-accurate or F16);
    // attention_type: the ViT attention (F32-accurate, as the reference's
    // GGML_PREC_F32, or fp16 operands).
    HipVisionEncoder(HipBackend& backend, const DeviceWeights& weights, VisionParameters params,
                     int32_t columns_type = SAMHIP_TYPE_F32, int32_t attention_type = SAMHIP_TYPE_F32)
        : be_(&backend), p_(std::move(params)) {
        p_.validate();
        const int E = p_.embed, G = p_.grid(), pg = p_.pos_grid(), D = p_.neck_dim;
        prefix_.version = SAMHIP_ABI_VERSION;
        prefix_.image_size = p_.image_size;
        prefix_.patch = p_.patch;
        prefix_.embed = E;
        prefix_.pos_grid = pg;
        prefix_.patch_w = f32(weights, "vit.patch_embed.proj.weight", {p_.patch, p_.patch, 3, E});
        prefix_.pos_embed = f32(weights, "vit.pos_embed", {E, pg, pg});
        prefix_.ln_pre_w = f32(weights, "vit.ln_pre.weight", {E});
        prefix_.ln_pre_b = f32(weights, "vit.ln_pre.bias", {E});
        for (int i = 0; i < p_.blocks; ++i) {
            const std::string b = "vit.blocks." + std::to_string(i);
            const bool global = p_.is_global(i);
            samhip_vit_block_desc d{};
            d.version = SAMHIP_ABI_VERSION;
            d.embed = E;
            d.heads = p_.heads;
            d.mlp = p_.mlp;
            d.grid_w = G;
            d.grid_h = G;
            d.window = global ? 0 : p_.window;
            d.norm1_w = f32(weights, b + ".norm1.weight", {E});
            d.norm1_b = f32(weights, b + ".norm1.bias", {E});
            d.norm2_w = f32(weights, b + ".norm2.weight", {E});
            d.norm2_b = f32(weights, b + ".norm2.bias", {E});
            d.qkv_w = linear(weights, b + ".attn.qkv.weight", E, 3 * E);
            d.qkv_b = f32(weights, b + ".attn.qkv.bias", {3 * E});
            d.proj_w = linear(weights, b + ".attn.proj.weight", E, E);
            d.proj_b = f32(weights, b + ".attn.proj.bias", {E});
            d.fc1_w = linear(weights, b + ".mlp.lin1.weight", E, p_.mlp);
            d.fc1_b = f32(weights, b + ".mlp.lin1.bias", {p_.mlp});
            d.fc2_w = linear(weights, b + ".mlp.lin2.weight", p_.mlp, E);
            d.fc2_b = f32(weights, b + ".mlp.lin2.bias", {E});
            d.attention_type = attention_type;
            const int tokens = global ? G * G : p_.window * p_.window;
            d.freqs_cis = f32(weights, b + ".attn.freqs_cis", {2, 32, tokens});
            blocks_.push_back(d);
        }
        const std::string n = "neck.det.";
        const int mid = neck_mid(weights);
        neck_.version = SAMHIP_ABI_VERSION;
        neck_.grid = G;
        neck_.embed = E;
        neck_.mid = mid;
        neck_.dim = D;
        neck_.columns_type = columns_type;
        auto conv = [&](samhip_neck_scale& s, const std::string& pre, int cin) {
            s.conv1x1_w = f32(weights, pre + "conv_1x1.weight", {1, 1, cin, D});
            s.conv1x1_b = f32(weights, pre + "conv_1x1.bias", {D});
            s.conv3x3_w = f32(weights, pre + "conv_3x3.weight", {3, 3, D, D});
            s.conv3x3_b = f32(weights, pre + "conv_3x3.bias", {D});
        };
        samhip_neck_scale* s = neck_.scales;
        s[0].deconv1_w = f32(weights, n + "0.dconv_2x2_0.weight", {2, 2, mid, E});
        s[0].deconv1_b = f32(weights, n + "0.dconv_2x2_0.bias", {mid});
        s[0].deconv2_w = f32(weights, n + "0.dconv_2x2_1.weight", {2, 2, D, mid});
        s[0].deconv2_b = f32(weights, n + "0.dconv_2x2_1.bias", {D});
        conv(s[0], n + "0.", D);
        s[1].deconv1_w = f32(weights, n + "1.dconv_2x2.weight", {2, 2, mid, E});
        s[1].deconv1_b = f32(weights, n + "1.dconv_2x2.bias", {mid});
        conv(s[1], n + "1.", mid);
        conv(s[2], n + "2.", E);
        has_level3_ = weights.has(n + "3.conv_1x1.weight");
        if (has_level3_) conv(s[3], n + "3.", E);
        x_ = static_cast<float*>(be_->alloc(size_t(G) * G * E * 4));
    }
    HipVisionEncoder(const HipVisionEncoder&) = delete;
    HipVisionEncoder& operator=(const HipVisionEncoder&) = delete;
    ~HipVisionEncoder() {
        if (x_) samhip_buffer_free(be_->handle(), x_);
    }

    const VisionParameters& parameters() const { return p_; }
    // side of neck level i (0..3): 4, 2, 1 and 1/2 times the grid
    int level_side(int level) const { return (4 * p_.grid()) >> level; }
    // The ViT output of the last encode (device F32 [grid*grid][embed]).
    const float* features() const { return x_; }

    // image: device F32 ggml {image_size, image_size, 3} (preprocessed
    // planes); levels[i] (device F32 [side*side][neck_dim], 16-byte aligned)
    // receive the neck maps, NULL levels are skipped.  Stream-ordered on the
    // backend's stream; synchronize before reading the results on the host.
    void encode(const float* image, float* const levels[4]) {
        if (levels[3] && !has_level3_) throw std::runtime_error("checkpoint has no neck level 3 weights");
        check_status(samhip_vit_prefix(be_->handle(), &prefix_, image, x_));
        for (const auto& d : blocks_) check_status(samhip_vit_block(be_->handle(), &d, x_));
        check_status(samhip_vit_neck(be_->handle(), &neck_, x_, levels[0], levels[1], levels[2], levels[3]));
    }

private:
    static const DeviceTensor& tensor(const DeviceWeights& w, const std::string& name, std::vector<int64_t> dims) {
        const DeviceTensor& t = w[name];
        while (dims.size() > 1 && dims.back() == 1) dims.pop_back();
        if (t.info.dims != dims) throw std::runtime_error("SAM 3 tensor shape differs from the encoder's: " + name);
        return t;
    }
    static const float* f32(const DeviceWeights& w, const std::string& name, std::vector<int64_t> dims) {
        const DeviceTensor& t = tensor(w, name, std::move(dims));
        if (t.info.type != SAMHIP_TYPE_F32) throw std::runtime_error("SAM 3 encoder tensor must be F32: " + name);
        return static_cast<const float*>(t.data);
    }
    static samhip_tensor linear(const DeviceWeights& w, const std::string& name, int K, int N) {
        const DeviceTensor& t = tensor(w, name, {K, N});
        if (!is_quantized_linear_type(t.info.type))
            throw std::runtime_error("SAM 3 encoder linear must be Q8_0 or a K-quant: " + name);
        return t.view();
    }
    // the transposed convolutions' width (512 in SAM 3), from the first one's shape
    int neck_mid(const DeviceWeights& w) const {
        const DeviceTensor& t = w["neck.det.0.dconv_2x2_0.weight"];
        if (t.info.dims.size() != 4) throw std::runtime_error("SAM 3 tensor shape differs from the encoder's: neck");
        return int(t.info.dims[2]);
    }

    HipBackend* be_;
    VisionParameters p_;
    samhip_vit_prefix_desc prefix_{};
    std::vector<samhip_vit_block_desc> blocks_;
    samhip_vit_neck_desc neck_{};
    bool has_level3_ = false;
    float* x_ = nullptr;
};

}  // namespace sam
