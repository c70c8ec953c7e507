// Core host types of the MI355X EdgeFM runtime: dtype/device enums with the
// reference's ordinals, a tensor handle (non-owning views and owning device/host
// buffers), the request/response types and the exception hierarchy
// (include/edge-fm/core.h:12-477 of the reference).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "edgefm_hip.h"

namespace edge_fm {

enum class Device { CPU, GPU };

// Same ordinals as the reference (core.h:17-25); shape_sig strings use them.
enum class DType { Float32, Float16, BFloat16, Int32, Int64, UInt8, Int8 };

enum class MemoryOwnership { ViewExternal, OwnCpuMalloc, OwnCudaMalloc, OwnCudaPool };

enum class ModelStage { Prefill, Decode };

size_t dtype_size(DType d);
DType dtype_from_string(const std::string& s);
std::string dtype_name(DType d);

// ---- exceptions (core.h:219-407) ----
class Error : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};
struct InvalidRequestError : Error { using Error::Error; };
struct DeviceError : Error { using Error::Error; };
struct InvalidArgumentError : Error { using Error::Error; };
struct ConfigurationError : Error { using Error::Error; };
struct ModelNotLoadedError : Error { using Error::Error; };
struct OutOfMemoryError : Error { using Error::Error; };
struct InternalError : Error { using Error::Error; };

template <class E>
inline void check(bool cond, const std::string& msg) {
    if (!cond) throw E(msg);
}

void hip_check(hipError_t e, const std::string& what);
// Map an edgefm_hip status code to the reference's exception types.
void efm_check(int status, const std::string& what);

class Tensor {
public:
    Tensor() = default;

    static Tensor view(void* data, std::vector<int64_t> shape, DType dtype, Device device, int32_t device_id = 0);
    static Tensor empty(std::vector<int64_t> shape, DType dtype, Device device, int32_t device_id = 0);
    static Tensor zeros(std::vector<int64_t> shape, DType dtype, Device device, int32_t device_id = 0);
    static Tensor clone_from(const void* src, std::vector<int64_t> shape, DType dtype, Device src_device,
                             int32_t src_device_id, Device dst_device, int32_t dst_device_id,
                             hipStream_t stream = nullptr);

    void* data_ptr() const { return data_; }
    const std::vector<int64_t>& shape() const { return shape_; }
    DType dtype() const { return dtype_; }
    std::pair<Device, int32_t> device() const { return {device_, device_id_}; }
    bool empty() const { return data_ == nullptr; }
    bool owns() const { return static_cast<bool>(owner_); }
    int64_t numel() const;
    size_t nbytes() const { return (size_t)numel() * dtype_size(dtype_); }
    // Same storage, new shape (element count must match).
    Tensor reshape(std::vector<int64_t> shape) const;
    // View of the leading elements of this buffer with a new shape (element count must
    // not exceed this tensor's).
    Tensor prefix_view(std::vector<int64_t> shape) const;

private:
    void* data_ = nullptr;
    std::vector<int64_t> shape_;
    DType dtype_ = DType::Float32;
    Device device_ = Device::CPU;
    int32_t device_id_ = 0;
    std::shared_ptr<void> owner_;
};

struct Request {
    Request(int32_t request_id, std::vector<int32_t> token_ids) : request_id(request_id), token_ids(std::move(token_ids)) {}
    int32_t request_id = 0;
    std::vector<int32_t> token_ids;
    // Optional custom embedding rows inserted for ids in [embed_token_id, +rows).
    Tensor embedding;
    int32_t embed_token_id = -1;
    // Optional M-RoPE position ids [3, seq_len] and the last position triplet.
    Tensor position_ids;
    std::vector<int32_t> mrope_last_pos;
    std::vector<int32_t> stop_token_ids;
    bool ignore_stop_tokens = false;

    bool has_embedding() const { return !embedding.empty(); }
    bool has_position_ids() const { return !position_ids.empty(); }
};

struct Response {
    std::vector<int32_t> token_ids;
};

}  // namespace edge_fm
