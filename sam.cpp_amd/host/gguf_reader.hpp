// GGUF v3 reader and device upload of SAM 3 checkpoints for the HIP backend.
//
// A self-contained parser of the GGUF container (ggml's gguf.c is not linked)
// that accepts exactly the files SAM.cpp's GgufReader accepts
// (src/io/gguf_reader.hpp:36-190) and rejects the same malformed ones
// (tests/api/test_contracts.cpp:364-460):
//   * magic "GGUF", little-endian version 3, 1..4096 tensors, <= 256 keys,
//     metadata parsed within min(file size, 16 MiB), general.alignment (when
//     present) a u32 equal to 32;
//   * tensor ranks 1..4, every dimension positive, no element or byte
//     overflow, row width a multiple of the type's block, byte count =
//     elements / block * type size;
//   * tensors stored back to back in table order at 32-byte aligned offsets,
//     zero padding after each one, no byte after the last one;
//   * keys and tensor names nonempty and unique, no string holding a NUL,
//     tensor names shorter than 64 bytes, and the metadata prefix
//     byte-identical to its canonical serialization (no alternative
//     encoding of the same content, e.g. a trailing dimension of 1).
// DeviceWeights then validates quantized payloads with
// samhip_validate_quantized_payload (src/models/sam3/weights.hpp:384-425) and
// uploads the bytes unchanged; expected_tensor_types resolves the storage
// profile's per-tensor types (src/models/sam3/weights.hpp:537-623).
#pragma once

#include "sam_hip.hpp"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace sam {

// GGUF metadata value types (gguf_type in ggml's gguf.h).
enum class GgufType : uint32_t {
    U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, Bool = 7, String = 8, Array = 9, U64 = 10,
    I64 = 11, F64 = 12
};

struct GgufValue {
    GgufType type = GgufType::U8;
    GgufType array_type = GgufType::U8;   // element type of an Array
    uint64_t bits = 0;                     // scalar: raw little-endian bits (floats too)
    std::string text;                      // String
    std::vector<uint64_t> elements;        // Array of scalars: raw bits per element
    std::vector<std::string> strings;      // Array of String
    uint64_t count() const { return array_type == GgufType::String ? strings.size() : elements.size(); }
};

struct GgufTensorInfo {
    std::string name;
    std::vector<int64_t> dims;   // trailing 1s removed (at least one dimension)
    int64_t ne[4] = {1, 1, 1, 1};
    int32_t type = 0;
    uint64_t offset = 0;         // absolute file offset of the data
    uint64_t size_bytes = 0;
};

// Block elements and bytes of the GGML storage types (ggml type traits).
inline bool ggml_block(int32_t type, uint64_t& elems, uint64_t& bytes) {
    struct Row { int32_t type; uint32_t elems, bytes; };
    static const Row table[] = {
        {0, 1, 4},      {1, 1, 2},      {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},
        {8, 32, 34},    {9, 32, 36},    {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
        {14, 256, 210}, {15, 256, 292}, {24, 1, 1},     {25, 1, 2},     {26, 1, 4},     {27, 1, 8},
        {28, 1, 8},     {30, 1, 2},
    };
    for (const Row& r : table)
        if (r.type == type) {
            elems = r.elems;
            bytes = r.bytes;
            return true;
        }
    return false;
}

class GgufReader {
public:
    static constexpr uint64_t kMetadataLimit = 16u * 1024u * 1024u;
    static constexpr uint64_t kAlignment = 32;
    static constexpr size_t kMaxTensorName = 63;

    explicit GgufReader(const std::string& path) : stream_(path, std::ios::binary) {
        if (!stream_) throw std::runtime_error("cannot open SAM checkpoint: " + path);
        stream_.seekg(0, std::ios::end);
        const auto length = stream_.tellg();
        if (length < 0) throw std::runtime_error("cannot determine SAM checkpoint size");
        size_ = uint64_t(length);
        meta_.resize(size_t(std::min<uint64_t>(size_, kMetadataLimit)));
        read(0, meta_.data(), meta_.size());
        if (size_ < 4) throw std::runtime_error("truncated GGUF checkpoint header");
        if (std::memcmp(meta_.data(), "GGUF", 4) != 0)
            throw std::runtime_error("unsupported checkpoint: expected GGUF; reconvert the original .pt checkpoint "
                                     "with tools/convert_sam3.py, rather than loading a legacy .ggml file");
        if (size_ < 24) throw std::runtime_error("truncated GGUF checkpoint header");
        pos_ = 4;
        if (u32() != 3) throw std::runtime_error("SAM checkpoints require little-endian GGUF v3");
        const uint64_t tensor_count = u64(), key_count = u64();
        if (tensor_count == 0 || tensor_count > 4096 || key_count > 256)
            throw std::runtime_error("GGUF tensor or metadata key count exceeds checkpoint limits");
        for (uint64_t i = 0; i < key_count; ++i) {
            std::string key = str(false);
            const GgufType t = GgufType(u32());
            GgufValue v = parse_value(t);
            if (!keys_.emplace(key, std::move(v)).second) throw std::runtime_error("ambiguous GGUF metadata key: " + key);
            key_order_.push_back(std::move(key));
        }
        auto al = keys_.find("general.alignment");
        if (al != keys_.end() && (al->second.type != GgufType::U32 || al->second.bits != kAlignment))
            throw std::runtime_error("SAM GGUF checkpoints require 32-byte alignment");
        std::vector<uint64_t> relative;
        for (uint64_t i = 0; i < tensor_count; ++i) {
            GgufTensorInfo t;
            t.name = str(false);
            if (t.name.size() > kMaxTensorName) throw std::runtime_error("GGUF tensor name is too long: " + t.name);
            const uint32_t nd = u32();
            if (nd == 0 || nd > 4) throw std::runtime_error("invalid GGUF tensor rank: " + t.name);
            uint64_t elements = 1;
            for (uint32_t d = 0; d < nd; ++d) {
                const uint64_t n = u64();
                if (n == 0 || n > uint64_t(INT64_MAX) || elements > uint64_t(INT64_MAX) / n)
                    throw std::runtime_error("invalid or overflowing GGUF tensor dimensions: " + t.name);
                elements *= n;
                t.ne[d] = int64_t(n);
            }
            t.dims.assign(t.ne, t.ne + 4);
            while (t.dims.size() > 1 && t.dims.back() == 1) t.dims.pop_back();
            t.type = int32_t(u32());
            uint64_t block = 0, block_bytes = 0;
            if (!ggml_block(t.type, block, block_bytes))
                throw std::runtime_error("unsupported GGUF tensor type: " + t.name);
            if (uint64_t(t.ne[0]) % block != 0)
                throw std::runtime_error("GGUF tensor row width is not quantization-block aligned: " + t.name);
            if (elements / block > UINT64_MAX / block_bytes)
                throw std::runtime_error("invalid or overflowing GGUF tensor byte count: " + t.name);
            t.size_bytes = elements / block * block_bytes;
            relative.push_back(u64());
            for (const auto& o : tensors_)
                if (o.name == t.name) throw std::runtime_error("duplicate GGUF tensor name: " + t.name);
            tensors_.push_back(std::move(t));
        }
        data_offset_ = (pos_ + kAlignment - 1) / kAlignment * kAlignment;
        if (data_offset_ > size_) throw std::runtime_error("truncated GGUF data section");
        const uint64_t available = size_ - data_offset_;
        uint64_t expected = 0;
        for (size_t i = 0; i < tensors_.size(); ++i) {
            auto& t = tensors_[i];
            const uint64_t rel = relative[i];
            const uint64_t padding = (kAlignment - t.size_bytes % kAlignment) % kAlignment;
            if (rel != expected || rel > available || t.size_bytes > available - rel ||
                padding > available - rel - t.size_bytes)
                throw std::runtime_error("overlapping, overflowing or truncated GGUF tensor range: " + t.name);
            t.offset = data_offset_ + rel;
            if (padding) {
                char pad[kAlignment] = {};
                read(t.offset + t.size_bytes, pad, size_t(padding));
                if (std::any_of(pad, pad + padding, [](char c) { return c != 0; }))
                    throw std::runtime_error("nonzero GGUF tensor padding: " + t.name);
            }
            expected = rel + t.size_bytes + padding;
        }
        if (expected != available) throw std::runtime_error("unexpected data after GGUF tensor blob");
        validate_canonical();
    }

    uint64_t size() const { return size_; }
    uint64_t data_offset() const { return data_offset_; }
    const std::vector<GgufTensorInfo>& tensors() const { return tensors_; }
    const GgufTensorInfo& tensor(const std::string& name) const {
        for (const auto& t : tensors_)
            if (t.name == name) return t;
        throw std::runtime_error("missing GGUF tensor: " + name);
    }

    // Typed metadata getters (GgufReader::key / u32 / string / array).
    bool has(const std::string& key) const { return keys_.count(key) != 0; }
    const GgufValue& value(const std::string& key, GgufType type) const {
        auto it = keys_.find(key);
        if (it == keys_.end() || it->second.type != type)
            throw std::runtime_error("missing or incompatible GGUF metadata: " + key);
        return it->second;
    }
    uint32_t u32(const std::string& key) const { return uint32_t(value(key, GgufType::U32).bits); }
    std::string string(const std::string& key, size_t maximum = 2048) const {
        return bounded_string(value(key, GgufType::String).text, maximum, key);
    }
    const GgufValue& array(const std::string& key, GgufType type, uint64_t count) const {
        const GgufValue& v = value(key, GgufType::Array);
        if (v.array_type != type || v.count() != count) throw std::runtime_error("incompatible GGUF array: " + key);
        return v;
    }
    static std::string bounded_string(const std::string& s, size_t maximum, const std::string& name) {
        if (s.empty() || s.size() > maximum) throw std::runtime_error("invalid or oversized GGUF string: " + name);
        return s;
    }

    void read(uint64_t offset, void* out, size_t bytes) {
        if (offset > size_ || bytes > size_ - offset) throw std::runtime_error("invalid or truncated GGUF file range");
        stream_.clear();
        stream_.seekg(std::streamoff(offset));
        stream_.read(static_cast<char*>(out), std::streamsize(bytes));
        if (!stream_) throw std::runtime_error("GGUF checkpoint changed or became unreadable");
    }
    std::vector<uint8_t> tensor_bytes(const GgufTensorInfo& t) {
        std::vector<uint8_t> out(size_t(t.size_bytes));
        read(t.offset, out.data(), out.size());
        return out;
    }

private:
    // -- little-endian cursor over the metadata prefix -------------------------
    uint64_t remaining() const { return pos_ <= meta_.size() ? meta_.size() - pos_ : 0; }
    void need(uint64_t n) const {
        if (n > remaining()) throw std::runtime_error("invalid, truncated or oversized GGUF metadata");
    }
    uint64_t le(int bytes) {
        need(uint64_t(bytes));
        uint64_t v = 0;
        for (int i = 0; i < bytes; ++i) v |= uint64_t(uint8_t(meta_[size_t(pos_) + i])) << (8 * i);
        pos_ += uint64_t(bytes);
        return v;
    }
    uint32_t u32() { return uint32_t(le(4)); }
    uint64_t u64() { return le(8); }
    // Keys and tensor names must be nonempty; values may be empty (the typed
    // getter rejects an empty string).
    std::string str(bool allow_empty) {
        const uint64_t n = u64();
        need(n);
        std::string s(meta_.data() + pos_, size_t(n));
        pos_ += n;
        if ((!allow_empty && s.empty()) || s.find('\0') != std::string::npos)
            throw std::runtime_error("empty GGUF key or name, or a string holding a NUL");
        return s;
    }
    static int scalar_bytes(GgufType t) {
        switch (t) {
            case GgufType::U8: case GgufType::I8: case GgufType::Bool: return 1;
            case GgufType::U16: case GgufType::I16: return 2;
            case GgufType::U32: case GgufType::I32: case GgufType::F32: return 4;
            case GgufType::U64: case GgufType::I64: case GgufType::F64: return 8;
            default: return 0;
        }
    }
    uint64_t scalar(GgufType t) {
        const uint64_t v = le(scalar_bytes(t));
        if (t == GgufType::Bool && v > 1) throw std::runtime_error("invalid GGUF bool value");
        return v;
    }
    GgufValue parse_value(GgufType t) {
        GgufValue v;
        v.type = t;
        if (t == GgufType::String) {
            v.text = str(true);
        } else if (t == GgufType::Array) {
            v.array_type = GgufType(u32());
            const uint64_t n = u64();
            const int width = v.array_type == GgufType::String ? 8 : scalar_bytes(v.array_type);
            if (width == 0) throw std::runtime_error("unsupported GGUF array element type");
            if (n > remaining() / uint64_t(width)) throw std::runtime_error("invalid, truncated or oversized GGUF array");
            for (uint64_t i = 0; i < n; ++i) {
                if (v.array_type == GgufType::String) v.strings.push_back(str(true));
                else v.elements.push_back(scalar(v.array_type));
            }
        } else if (scalar_bytes(t) != 0) {
            v.bits = scalar(t);
        } else {
            throw std::runtime_error("unsupported GGUF metadata value type");
        }
        return v;
    }

    // -- canonical serialization ------------------------------------------------
    static void put(std::string& o, uint64_t v, int bytes) {
        for (int i = 0; i < bytes; ++i) o.push_back(char((v >> (8 * i)) & 0xff));
    }
    static void put_str(std::string& o, const std::string& s) {
        put(o, s.size(), 8);
        o += s;
    }
    void validate_canonical() const {
        std::string o = "GGUF";
        put(o, 3, 4);
        put(o, tensors_.size(), 8);
        put(o, key_order_.size(), 8);
        for (const auto& key : key_order_) {
            const GgufValue& v = keys_.at(key);
            put_str(o, key);
            put(o, uint32_t(v.type), 4);
            if (v.type == GgufType::String) {
                put_str(o, v.text);
            } else if (v.type == GgufType::Array) {
                put(o, uint32_t(v.array_type), 4);
                put(o, v.count(), 8);
                for (const auto& s : v.strings) put_str(o, s);
                for (uint64_t x : v.elements) put(o, x, scalar_bytes(v.array_type));
            } else {
                put(o, v.bits, scalar_bytes(v.type));
            }
        }
        for (const auto& t : tensors_) {
            put_str(o, t.name);
            put(o, uint32_t(t.dims.size()), 4);
            for (int64_t d : t.dims) put(o, uint64_t(d), 8);
            put(o, uint32_t(t.type), 4);
            put(o, t.offset - data_offset_, 8);
        }
        while (o.size() % kAlignment) o.push_back('\0');
        if (o.size() != data_offset_ || std::memcmp(o.data(), meta_.data(), o.size()) != 0)
            throw std::runtime_error("noncanonical GGUF metadata, string or tensor dimensions");
    }

    std::ifstream stream_;
    std::vector<char> meta_;
    uint64_t size_ = 0, pos_ = 0, data_offset_ = 0;
    std::map<std::string, GgufValue> keys_;
    std::vector<std::string> key_order_;
    std::vector<GgufTensorInfo> tensors_;
};

// ---------------------------------------------------------------------------
// Storage profile of a SAM 3 image checkpoint
// ---------------------------------------------------------------------------

// Per-tensor GGUF type the checkpoint's storage profile requires, or -1 where
// this layer does not constrain it.  Schema 3 (image-*linear-*) and schema 4
// (image-full-* / image-modules-* with sam.quantization.modules) follow
// src/models/sam3/weights.hpp:537-575 and :600-620: the profile must exist,
// general.file_type must be the profile's, general.quantization_version must
// be 2.  Unquantized schemas (1, 2) and the mixed schemas (5-7, whose
// precision policy is a separate document) impose no per-tensor type here;
// their quantized payloads are still validated by DeviceWeights::load.
inline std::function<int32_t(const GgufTensorInfo&)> expected_tensor_types(const GgufReader& reader) {
    const uint32_t schema = reader.u32("sam.schema_version");
    if (schema < 1 || schema > 7) throw std::runtime_error("unsupported SAM GGUF schema version");
    if (schema >= 3 && !reader.has("sam.storage_profile"))
        throw std::runtime_error("quantized SAM GGUF is missing its storage profile");
    const uint32_t file_type = reader.u32("general.file_type");
    if (schema == 3) {
        const std::string name = reader.string("sam.storage_profile");
        const policy::ImageQuantizationProfile* p = policy::image_quantization_profile(name);
        if (!p) throw std::runtime_error("unsupported SAM GGUF quantization profile (storage profile " + name + ")");
        if (file_type != p->file_type)
            throw std::runtime_error("SAM GGUF file type does not match its quantization profile");
        if (reader.u32("general.quantization_version") != 2)
            throw std::runtime_error("unsupported GGML quantization version");
        return [p](const GgufTensorInfo& t) { return policy::image_quantized_tensor_type(t.name, t.dims, *p); };
    }
    if (schema == 4) {
        const std::string name = reader.string("sam.storage_profile");
        const policy::ModularImageQuantizationProfile* p = policy::modular_image_quantization_profile(name);
        if (!p) throw std::runtime_error("unsupported modular SAM GGUF quantization profile (storage profile " + name + ")");
        const std::vector<std::string> modules =
            policy::parse_image_quantization_modules(reader.string("sam.quantization.modules", 64));
        if (p->full_preset && modules.size() != policy::module_order().size())
            throw std::runtime_error("SAM modular profile does not match its canonical module list");
        if (file_type != p->file_type)
            throw std::runtime_error("SAM GGUF file type does not match its modular profile");
        if (reader.u32("general.quantization_version") != 2)
            throw std::runtime_error("unsupported GGML quantization version");
        return [p, modules](const GgufTensorInfo& t) {
            return policy::image_modular_quantized_tensor_type(t.name, t.dims, *p, modules);
        };
    }
    if (schema <= 2) {
        if (file_type > 1) throw std::runtime_error("SAM GGUF precision must be F32 or mixed F16");
        if (reader.has("sam.storage_profile") &&
            (schema != 2 || file_type != 1 || reader.string("sam.storage_profile") != "visual-tracker-f32-v1"))
            throw std::runtime_error("unsupported SAM GGUF storage profile");
    } else if (reader.u32("general.quantization_version") != 2) {
        throw std::runtime_error("unsupported GGML quantization version");
    }
    return [](const GgufTensorInfo&) { return int32_t(-1); };
}

// ---------------------------------------------------------------------------
// Upload to the HIP backend
// ---------------------------------------------------------------------------

inline bool is_quantized_linear_type(int32_t type) {
    return type == SAMHIP_TYPE_Q8_0 || type == SAMHIP_TYPE_Q4_K || type == SAMHIP_TYPE_Q5_K || type == SAMHIP_TYPE_Q6_K;
}

// Checks a quantized tensor's bytes before they reach a device: finite,
// bounded block scales (samhip_validate_quantized_payload); other types pass.
inline void validate_tensor_payload(const GgufTensorInfo& t, const std::vector<uint8_t>& bytes) {
    if (!is_quantized_linear_type(t.type)) return;
    const int64_t rows = t.ne[1] * t.ne[2] * t.ne[3];
    if (samhip_validate_quantized_payload(t.type, t.ne[0], rows, bytes.data(), bytes.size()) != SAMHIP_OK)
        throw std::runtime_error(samhip_message() + ": " + t.name);
}

// A tensor resident on the device, owned by the DeviceWeights that holds it.
struct DeviceTensor {
    GgufTensorInfo info;
    void* data = nullptr;
    // ggml view of the whole tensor: nb[0] = block bytes, nb[1] = row bytes.
    samhip_tensor view() const {
        uint64_t block = 1, block_bytes = 4;
        ggml_block(info.type, block, block_bytes);
        samhip_tensor t{};
        t.type = info.type;
        for (int d = 0; d < 4; ++d) t.ne[d] = info.ne[d];
        t.nb[0] = size_t(block_bytes);
        t.nb[1] = size_t(uint64_t(info.ne[0]) / block * block_bytes);
        t.nb[2] = t.nb[1] * size_t(info.ne[1]);
        t.nb[3] = t.nb[2] * size_t(info.ne[2]);
        t.data = data;
        return t;
    }
};

// Device copies of a checkpoint's tensors; frees them on destruction.
class DeviceWeights {
public:
    explicit DeviceWeights(HipBackend& backend) : backend_(&backend) {}
    DeviceWeights(const DeviceWeights&) = delete;
    DeviceWeights& operator=(const DeviceWeights&) = delete;
    ~DeviceWeights() {
        for (auto& kv : tensors_) samhip_buffer_free(backend_->handle(), kv.second.data);
    }

    // Uploads the tensors `select` accepts (all when empty) byte for byte.
    // Before the first upload every selected tensor's type is checked
    // against `expected_type` (when given; -1 = unconstrained).  Each
    // quantized payload is validated (finite, bounded scales) before its
    // upload; a failure throws and leaves the tensors uploaded so far owned
    // by this object.
    void load(GgufReader& reader, const std::function<bool(const GgufTensorInfo&)>& select = {},
              const std::function<int32_t(const GgufTensorInfo&)>& expected_type = {}) {
        std::vector<const GgufTensorInfo*> chosen;
        for (const auto& t : reader.tensors()) {
            if (select && !select(t)) continue;
            if (tensors_.count(t.name)) throw std::runtime_error("tensor already loaded: " + t.name);
            if (expected_type) {
                const int32_t want = expected_type(t);
                if (want >= 0 && want != t.type)
                    throw std::runtime_error("incompatible SAM 3 tensor precision: " + t.name + " is " +
                                             type_name(t.type) + ", its storage profile requires " + type_name(want));
            }
            chosen.push_back(&t);
        }
        for (const auto* t : chosen) {
            std::vector<uint8_t> bytes = reader.tensor_bytes(*t);
            validate_tensor_payload(*t, bytes);
            DeviceTensor d;
            d.info = *t;
            d.data = backend_->alloc(bytes.size());
            tensors_.emplace(t->name, d);
            backend_->upload(d.data, bytes.data(), bytes.size());
            bytes_ += bytes.size();
        }
    }
    bool has(const std::string& name) const { return tensors_.count(name) != 0; }
    const DeviceTensor& operator[](const std::string& name) const {
        auto it = tensors_.find(name);
        if (it == tensors_.end()) throw std::runtime_error("tensor not loaded: " + name);
        return it->second;
    }
    size_t count() const { return tensors_.size(); }
    uint64_t bytes() const { return bytes_; }

private:
    HipBackend* backend_;
    std::map<std::string, DeviceTensor> tensors_;
    uint64_t bytes_ = 0;
};

}  // namespace sam
