// Portable attention interface of the reference (portable.rs:1-565,
// gpu_backend.rs:1-377) on top of libmslim_attn: exact little-endian K/V
// frames, the AttentionBackend plug-in contract, and the GPU backend that
// replaces the OpenCL QK/softmax/PV kernels with the fused gfx950 decode.
// Names, argument meaning and error kinds follow the reference.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "native.hpp"

namespace mslim {
namespace portable {

// portable.rs:11-35
enum class FloatFormat { Bf16, F16, F32 };
size_t bytes_per_element(FloatFormat f);
const char *label(FloatFormat f);
int format_code(FloatFormat f);  // MSLIM_ATTN_FORMAT_* (gpu_backend.rs:258-262)

// portable.rs:37-58: the error kinds and their Display texts.
class PortableError : public std::runtime_error {
public:
    enum class Kind { InvalidGeometry, ShapeMismatch, NonFinite, UnsupportedDevice, BackendFailure };
    PortableError(Kind kind, const std::string &message);
    Kind kind() const { return kind_; }
    const std::string &message() const { return message_; }

private:
    Kind kind_;
    std::string message_;
};

// portable.rs:60-175: a tensor's bytes (little-endian) with its dtype and
// shape; the bytes are copied in and never change.
class RawTensor {
public:
    static RawTensor from_le_bytes(FloatFormat dtype, std::vector<size_t> shape, std::vector<uint8_t> bytes);
    static RawTensor from_f32(std::vector<size_t> shape, const std::vector<float> &data);
    FloatFormat dtype() const { return dtype_; }
    const std::vector<size_t> &shape() const { return shape_; }
    const std::vector<uint8_t> &as_le_bytes() const { return *bytes_; }
    size_t len_bytes() const { return bytes_->size(); }
    std::vector<float> decode_f32() const;

private:
    RawTensor(FloatFormat d, std::vector<size_t> s, std::shared_ptr<const std::vector<uint8_t>> b)
        : dtype_(d), shape_(std::move(s)), bytes_(std::move(b)) {}
    FloatFormat dtype_;
    std::vector<size_t> shape_;
    std::shared_ptr<const std::vector<uint8_t>> bytes_;
};

// portable.rs:412-457
struct AttentionGeometry {
    size_t query_heads = 0, kv_heads = 0, head_dim = 0;
    static AttentionGeometry create(size_t query_heads, size_t kv_heads, size_t head_dim);
    size_t kv_head_for_query(size_t query_head) const;
    size_t query_elements() const { return query_heads * head_dim; }
    size_t kv_elements_per_token() const { return kv_heads * head_dim; }
    bool operator==(const AttentionGeometry &o) const {
        return query_heads == o.query_heads && kv_heads == o.kv_heads && head_dim == o.head_dim;
    }
};

class AttentionBackend;

// portable.rs:459-558: frames in [tokens, kv_heads, head_dim] order.
class ExactKvFrames {
public:
    explicit ExactKvFrames(AttentionGeometry geometry) : geometry_(geometry) {}
    void append(RawTensor key, RawTensor value);
    AttentionGeometry geometry() const { return geometry_; }
    size_t tokens() const { return tokens_; }
    bool is_empty() const { return frames_.empty(); }
    size_t payload_bytes() const;
    const std::vector<std::pair<RawTensor, RawTensor>> &frames() const { return frames_; }
    // SHA-256 over the domain string "mslim-portable-exact-kv-v1", then the
    // dtype, the shapes and the bytes of the stored K/V.
    std::string digest_sha256() const;
    std::vector<float> decode(const AttentionBackend &backend, const std::vector<float> &query) const;

private:
    AttentionGeometry geometry_;
    std::vector<std::pair<RawTensor, RawTensor>> frames_;
    size_t tokens_ = 0;
};

// portable.rs:561-565: pluggable kernel contract.
class AttentionBackend {
public:
    virtual ~AttentionBackend() = default;
    virtual const char *name() const = 0;
    virtual std::vector<float> decode(const ExactKvFrames &kv, const std::vector<float> &query) const = 0;
};

// gpu_backend.rs:21-32
struct GpuDeviceInfo {
    std::string name, vendor, arch, driver_version;
    uint32_t max_compute_units = 0;
    uint64_t reported_global_memory_bytes = 0;
    uint64_t max_allocation_bytes = 0;
};

// gpu_backend.rs:34-44, with the three OpenCL kernel times folded into one.
struct GpuTimings {
    double dispatch_ms = 0, kernel_ms = 0;
    size_t input_kv_bytes = 0, scratch_bytes = 0, output_bytes = 0;
};

// gpu_backend.rs:51-377 on MI355X.  Frames are uploaded into context-owned
// device buffers that are reused across calls.
class GpuBackend : public AttentionBackend {
public:
    GpuBackend();  // throws PortableError(UnsupportedDevice) without a gfx950 device
    const char *name() const override { return "mi355x-hip-fused-decode"; }
    std::vector<float> decode(const ExactKvFrames &kv, const std::vector<float> &query) const override;
    const GpuDeviceInfo &device_info() const { return info_; }
    std::optional<GpuTimings> last_timings() const;
    std::shared_ptr<NativeContext> context() const { return ctx_; }

private:
    std::shared_ptr<NativeContext> ctx_;
    GpuDeviceInfo info_;
    mutable std::mutex timings_mutex_;
    mutable std::optional<GpuTimings> last_;
};

}  // namespace portable
}  // namespace mslim
