#include "core.hpp"

#include <cstdlib>
#include <cstring>

namespace edge_fm {

size_t dtype_size(DType d) {
    switch (d) {
        case DType::Float32:
        case DType::Int32: return 4;
        case DType::Float16:
        case DType::BFloat16: return 2;
        case DType::Int64: return 8;
        case DType::UInt8:
        case DType::Int8: return 1;
    }
    return 0;
}

DType dtype_from_string(const std::string& s) {
    if (s == "fp32" || s == "float32") return DType::Float32;
    if (s == "fp16" || s == "float16") return DType::Float16;
    if (s == "bf16" || s == "bfloat16") return DType::BFloat16;
    if (s == "int32") return DType::Int32;
    if (s == "int64") return DType::Int64;
    if (s == "int8") return DType::Int8;
    if (s == "uint8") return DType::UInt8;
    throw ConfigurationError("Unsupported dtype: " + s);
}

std::string dtype_name(DType d) {
    switch (d) {
        case DType::Float32: return "float32";
        case DType::Float16: return "float16";
        case DType::BFloat16: return "bfloat16";
        case DType::Int32: return "int32";
        case DType::Int64: return "int64";
        case DType::UInt8: return "uint8";
        case DType::Int8: return "int8";
    }
    return "?";
}

void hip_check(hipError_t e, const std::string& what) {
    if (e != hipSuccess) {
        if (e == hipErrorOutOfMemory) throw OutOfMemoryError(what + ": " + hipGetErrorString(e));
        throw DeviceError(what + ": " + hipGetErrorString(e));
    }
}

void efm_check(int status, const std::string& what) {
    if (status == EFM_OK) return;
    const std::string msg = what + ": " + efm_last_error();
    switch (status) {
        case EFM_ERR_INVALID_ARGUMENT: throw InvalidRequestError(msg);
        case EFM_ERR_UNSUPPORTED: throw ConfigurationError(msg);
        case EFM_ERR_WORKSPACE: throw InternalError(msg);
        default: throw DeviceError(msg);
    }
}

int64_t Tensor::numel() const {
    int64_t n = 1;
    for (int64_t s : shape_) n *= s;
    return n;
}

Tensor Tensor::view(void* data, std::vector<int64_t> shape, DType dtype, Device device, int32_t device_id) {
    Tensor t;
    t.data_ = data;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.device_ = device;
    t.device_id_ = device_id;
    return t;
}

Tensor Tensor::empty(std::vector<int64_t> shape, DType dtype, Device device, int32_t device_id) {
    Tensor t = view(nullptr, std::move(shape), dtype, device, device_id);
    size_t bytes = std::max<size_t>(t.nbytes(), 16);
    bytes = (bytes + 255) & ~(size_t)255;
    if (device == Device::GPU) {
        int prev = 0;
        hip_check(hipGetDevice(&prev), "hipGetDevice");
        hip_check(hipSetDevice(device_id), "hipSetDevice");
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, bytes);
        hipSetDevice(prev);
        hip_check(e, "hipMalloc(" + std::to_string(bytes) + " bytes)");
        t.data_ = p;
        t.owner_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
    } else {
        void* p = std::aligned_alloc(256, bytes);
        if (p == nullptr) throw OutOfMemoryError("host allocation failed");
        t.data_ = p;
        t.owner_ = std::shared_ptr<void>(p, [](void* q) { std::free(q); });
    }
    return t;
}

Tensor Tensor::zeros(std::vector<int64_t> shape, DType dtype, Device device, int32_t device_id) {
    Tensor t = empty(std::move(shape), dtype, device, device_id);
    if (device == Device::GPU) hip_check(hipMemset(t.data_, 0, t.nbytes()), "hipMemset");
    else std::memset(t.data_, 0, t.nbytes());
    return t;
}

Tensor Tensor::clone_from(const void* src, std::vector<int64_t> shape, DType dtype, Device src_device,
                          int32_t src_device_id, Device dst_device, int32_t dst_device_id, hipStream_t stream) {
    (void)src_device_id;
    Tensor t = empty(std::move(shape), dtype, dst_device, dst_device_id);
    const size_t n = t.nbytes();
    if (n == 0) return t;
    if (src_device == Device::CPU && dst_device == Device::CPU) {
        std::memcpy(t.data_, src, n);
        return t;
    }
    hipMemcpyKind kind = src_device == Device::CPU ? hipMemcpyHostToDevice
                         : (dst_device == Device::CPU ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice);
    hip_check(hipMemcpyAsync(t.data_, src, n, kind, stream), "clone_from copy");
    hip_check(hipStreamSynchronize(stream), "clone_from sync");
    return t;
}

Tensor Tensor::reshape(std::vector<int64_t> shape) const {
    Tensor t = *this;
    t.shape_ = std::move(shape);
    check<InvalidArgumentError>(t.numel() == numel(), "reshape: element count mismatch");
    return t;
}

Tensor Tensor::prefix_view(std::vector<int64_t> shape) const {
    Tensor t = *this;
    t.shape_ = std::move(shape);
    check<InvalidArgumentError>(t.numel() <= numel(), "prefix_view: larger than the buffer");
    return t;
}

}  // namespace edge_fm
