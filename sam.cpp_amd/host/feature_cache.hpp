// Compact feature caches over the HIP backend: the device-side cast of a
// neck feature map to its cache type (ggml_cast to F16 or Q8_0,
// src/models/sam3/execution.hpp:76-83) and the host snapshot that keeps one
// representation of it (HostTensor, src/runtime/ggml/host_tensor.hpp:16-106):
// downloaded bytes with the reference's scale validation, a shape check that
// allows flattening but not a different row layout, re-upload with a
// device-side decode to F32 (cached_input's ggml_cast), and a host decode
// for F32 consumers and diagnostics.
#pragma once

#include "sam_hip.hpp"

#include <cstring>
#include <stdexcept>
#include <vector>

namespace sam {

// F32 value of IEEE binary16 bits.
inline float half_to_float(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {   // subnormal: renormalize
        exp = 113;
        while (!(man & 0x400u)) {
            man <<= 1;
            --exp;
        }
        bits = sign | (exp << 23) | ((man & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Storage type of neck level `level` (0..2) in a cache of `requested` type:
// the low-resolution level that drives fusion and detection stays F32 under
// Q8_0 (src/models/sam3/execution.hpp:75-79).
inline int32_t feature_cache_level_type(int level, int32_t requested) {
    return level == 2 && requested == SAMHIP_TYPE_Q8_0 ? SAMHIP_TYPE_F32 : requested;
}

class HipHostTensor {
public:
    // Casts device F32 rows [rows][row_elements] to `type` (F32, F16 or
    // Q8_0) on the device and keeps the bytes on the host.
    static HipHostTensor capture(HipBackend& be, const float* device_f32, int64_t rows, int64_t row_elements,
                                 int32_t type, int32_t q8_rounding = SAMHIP_Q8_ROUND_X86) {
        check_type(type, row_elements);
        if (rows <= 0 || row_elements <= 0) throw std::invalid_argument("invalid SAM cached tensor shape");
        HipHostTensor t;
        t.type_ = type;
        t.row_elements_ = row_elements;
        t.elements_ = size_t(rows) * size_t(row_elements);
        t.payload_.resize(size_t(rows) * row_size(type, row_elements));
        if (type == SAMHIP_TYPE_F32) {
            be.download(t.payload_.data(), device_f32, t.payload_.size());
        } else {
            Scratch s(be, t.payload_.size());
            check_status(samhip_quantize_rows(be.handle(), type, device_f32, size_t(row_elements) * 4, s.ptr, rows,
                                              row_elements, q8_rounding));
            be.download(t.payload_.data(), s.ptr, t.payload_.size());
        }
        t.validate_scales();
        return t;
    }

    // A snapshot from bytes already in the cache layout (validated).
    static HipHostTensor from_bytes(int32_t type, int64_t rows, int64_t row_elements, std::vector<uint8_t> bytes) {
        check_type(type, row_elements);
        if (rows <= 0 || row_elements <= 0 || bytes.size() != size_t(rows) * row_size(type, row_elements))
            throw std::runtime_error("invalid SAM cached tensor allocation, layout or type");
        HipHostTensor t;
        t.type_ = type;
        t.row_elements_ = row_elements;
        t.elements_ = size_t(rows) * size_t(row_elements);
        t.payload_ = std::move(bytes);
        t.validate_scales();
        return t;
    }

    int32_t type() const { return type_; }
    size_t elements() const { return elements_; }
    size_t size_bytes() const { return payload_.size(); }
    bool empty() const { return payload_.empty(); }
    const std::vector<uint8_t>& bytes() const { return payload_; }

    // Flattening spatial dimensions is permitted; changing the row layout is not.
    void validate_shape(int64_t d0, int64_t d1, int64_t d2, int64_t d3) const {
        size_t count = 1;
        for (int64_t d : {d0, d1, d2, d3}) {
            if (d <= 0) throw std::invalid_argument("invalid SAM cache input dimension");
            if (count > SIZE_MAX / size_t(d)) throw std::invalid_argument("SAM cached tensor shape overflows");
            count *= size_t(d);
        }
        if (empty() || count != elements_ || d0 != row_elements_)
            throw std::invalid_argument("SAM cache input shape or row layout differs");
    }

    // Uploads the stored bytes and decodes them to F32 rows at device_f32.
    void upload_f32(HipBackend& be, float* device_f32) const {
        if (empty()) throw std::runtime_error("no SAM cached tensor is available");
        const int64_t rows = int64_t(elements_ / size_t(row_elements_));
        if (type_ == SAMHIP_TYPE_F32) {
            be.upload(device_f32, payload_.data(), payload_.size());
            return;
        }
        Scratch s(be, payload_.size());
        be.upload(s.ptr, payload_.data(), payload_.size());
        check_status(samhip_dequantize_rows(be.handle(), type_, s.ptr, row_size(type_, row_elements_), device_f32, rows,
                                            row_elements_));
        be.synchronize();
    }

    // Host decode (ggml to_float of the stored type).
    std::vector<float> as_f32() const {
        if (empty()) throw std::runtime_error("no SAM cached tensor is available");
        std::vector<float> out(elements_);
        if (type_ == SAMHIP_TYPE_F32) {
            std::memcpy(out.data(), payload_.data(), payload_.size());
        } else if (type_ == SAMHIP_TYPE_F16) {
            for (size_t i = 0; i < elements_; ++i) {
                uint16_t h;
                std::memcpy(&h, payload_.data() + 2 * i, 2);
                out[i] = half_to_float(h);
            }
        } else {
            for (size_t b = 0; b < elements_ / 32; ++b) {
                const uint8_t* blk = payload_.data() + 34 * b;
                uint16_t h;
                std::memcpy(&h, blk, 2);
                const float d = half_to_float(h);
                for (int i = 0; i < 32; ++i) out[32 * b + i] = d * float(int8_t(blk[2 + i]));
            }
        }
        return out;
    }

private:
    struct Scratch {
        HipBackend& be;
        void* ptr;
        Scratch(HipBackend& b, size_t bytes) : be(b), ptr(b.alloc(bytes)) {}
        ~Scratch() { samhip_buffer_free(be.handle(), ptr); }
    };

    static void check_type(int32_t type, int64_t row_elements) {
        if (type != SAMHIP_TYPE_F32 && type != SAMHIP_TYPE_F16 && type != SAMHIP_TYPE_Q8_0)
            throw std::runtime_error("invalid SAM cached tensor allocation, layout or type");
        if (type != SAMHIP_TYPE_F32 && row_elements % 32)
            throw std::invalid_argument("SAM compact cache rows must hold whole 32-value groups");
    }
    static size_t row_size(int32_t type, int64_t row_elements) {
        return type == SAMHIP_TYPE_F32 ? size_t(row_elements) * 4
             : type == SAMHIP_TYPE_F16 ? size_t(row_elements) * 2 : size_t(row_elements) / 32 * 34;
    }
    // Overflow must not become an apparently valid compact snapshot: F16
    // stores each value directly, Q8_0 one half scale per block, which must
    // also be nonnegative (host_tensor.hpp:80-91).
    void validate_scales() const {
        if (type_ == SAMHIP_TYPE_F32) return;
        const size_t stride = type_ == SAMHIP_TYPE_F16 ? 2 : 34;
        for (size_t off = 0; off < payload_.size(); off += stride) {
            uint16_t bits;
            std::memcpy(&bits, payload_.data() + off, 2);
            if ((bits & 0x7c00u) == 0x7c00u || (type_ == SAMHIP_TYPE_Q8_0 && (bits & 0x8000u)))
                throw std::runtime_error("non-finite or invalid SAM compact cache value/scale");
        }
    }

    int32_t type_ = SAMHIP_TYPE_F32;
    int64_t row_elements_ = 0;
    size_t elements_ = 0;
    std::vector<uint8_t> payload_;
};

}  // namespace sam
