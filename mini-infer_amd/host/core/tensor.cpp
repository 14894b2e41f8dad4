// tensor.cpp -- HIP-backed implementation of mini_infer::Tensor.
#include "core/tensor.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>

namespace mini_infer {

const char* dtype_name(DType d) {
    switch (d) {
        case DType::FP32: return "fp32";
        case DType::FP16: return "fp16";
        case DType::BF16: return "bf16";
        case DType::INT32: return "int32";
        case DType::INT64: return "int64";
    }
    return "unknown";
}

namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string("HIP error in ") + what + ": " + hipGetErrorString(e));
}

// Makes `dev` current for the lifetime of the guard.
class DeviceGuard {
public:
    explicit DeviceGuard(Device dev) {
        if (!dev.is_cuda()) return;
        hip_check(hipGetDevice(&prev_), "hipGetDevice");
        if (prev_ != dev.index) {
            hip_check(hipSetDevice(dev.index), "hipSetDevice");
            switched_ = true;
        }
    }
    ~DeviceGuard() {
        if (switched_) (void)hipSetDevice(prev_);
    }

private:
    int prev_ = 0;
    bool switched_ = false;
};

// IEEE binary16 round-to-nearest-even of a finite or special fp32 value.
uint16_t half_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0));
    if (a >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return static_cast<uint16_t>(sign);
        const uint32_t shift = 126u - (a >> 23);
        const uint32_t sig = (a & 0x7fffffu) | 0x800000u;
        uint32_t q = sig >> shift;
        const uint32_t rem = sig & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return static_cast<uint16_t>(sign | q);
    }
    const uint32_t v = a - 0x38000000u;
    uint32_t q = v >> 13;
    const uint32_t rem = v & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return static_cast<uint16_t>(sign | q);
}

}  // namespace

Tensor::Tensor() = default;

Tensor::Tensor(std::vector<int64_t> shape, DType dtype, Device device)
    : shape_(std::move(shape)), dtype_(dtype), device_(device) {
    numel_ = 1;
    for (int64_t s : shape_) {
        if (s < 0) throw std::runtime_error("Tensor: negative dimension");
        numel_ *= s;
    }
    nbytes_ = static_cast<std::size_t>(numel_) * dtype_size(dtype_);
    compute_default_stride_();
    allocate_();
}

Tensor Tensor::empty(std::vector<int64_t> shape, DType dtype, Device device) {
    return Tensor(std::move(shape), dtype, device);
}

Tensor::Tensor(const Tensor& other)
    : shape_(other.shape_), stride_(other.stride_), numel_(other.numel_),
      nbytes_(other.nbytes_), dtype_(other.dtype_), device_(other.device_) {
    allocate_();
    if (nbytes_ > 0 && other.data_) copy_raw(other.data_, data_, nbytes_, other.device_, device_);
}

// Member-wise exchange: the building block of both assignments below
// (copy-and-swap), so each has one path that leaves *this either fully old
// or fully new.
void Tensor::swap_(Tensor& other) noexcept {
    using std::swap;
    swap(shape_, other.shape_);
    swap(stride_, other.stride_);
    swap(numel_, other.numel_);
    swap(nbytes_, other.nbytes_);
    swap(dtype_, other.dtype_);
    swap(device_, other.device_);
    swap(data_, other.data_);
    swap(owns_data_, other.owns_data_);
}

Tensor& Tensor::operator=(const Tensor& other) {
    if (this != &other) {
        Tensor copy(other);  // allocates and copies first: a failure leaves *this intact
        swap_(copy);
    }                        // copy now holds the old buffer and frees it
    return *this;
}

// The moved-from tensor is left empty (no shape, no buffer, not owning).
Tensor::Tensor(Tensor&& other) noexcept { swap_(other); }

Tensor& Tensor::operator=(Tensor&& other) noexcept {
    if (this != &other) {
        Tensor taken(std::move(other));
        swap_(taken);
    }  // taken holds the old buffer and frees it
    return *this;
}

Tensor::~Tensor() { release_(); }

void Tensor::compute_default_stride_() {
    stride_.assign(shape_.size(), 1);
    int64_t s = 1;
    for (int i = static_cast<int>(shape_.size()) - 1; i >= 0; --i) {
        stride_[i] = s;
        s *= shape_[i];
    }
}

void Tensor::allocate_() {
    if (nbytes_ == 0) return;
    if (device_.is_cuda()) {
        DeviceGuard g(device_);
        hip_check(hipMalloc(&data_, nbytes_), "hipMalloc");
    } else {
        data_ = ::operator new(nbytes_);
    }
    owns_data_ = true;
}

void Tensor::release_() {
    if (owns_data_ && data_) {
        if (device_.is_cuda()) {
            DeviceGuard g(device_);
            (void)hipFree(data_);
        } else {
            ::operator delete(data_);
        }
    }
    data_ = nullptr;
    owns_data_ = false;
}

bool Tensor::is_contiguous() const {
    if (stride_.size() != shape_.size()) return false;
    int64_t expected = 1;
    for (int i = static_cast<int>(shape_.size()) - 1; i >= 0; --i) {
        if (shape_[i] == 1) continue;
        if (stride_[i] != expected) return false;
        expected *= shape_[i];
    }
    return true;
}

void Tensor::copy_raw(const void* src, void* dst, std::size_t bytes, Device src_dev,
                      Device dst_dev) {
    if (bytes == 0) return;
    if (src_dev.is_cpu() && dst_dev.is_cpu()) {
        std::memcpy(dst, src, bytes);
        return;
    }
    hipMemcpyKind kind = hipMemcpyDeviceToDevice;
    if (src_dev.is_cpu()) kind = hipMemcpyHostToDevice;
    else if (dst_dev.is_cpu()) kind = hipMemcpyDeviceToHost;
    hip_check(hipMemcpy(dst, src, bytes, kind), "hipMemcpy");
}

Tensor Tensor::to(Device target) const {
    Tensor out(shape_, dtype_, target);
    if (nbytes_ > 0) copy_raw(data_, out.data_, nbytes_, device_, target);
    return out;
}

void Tensor::fill(float value) {
    if (nbytes_ == 0 || !data_) return;
    if (dtype_ != DType::FP32 && dtype_ != DType::FP16)
        throw std::runtime_error("Tensor::fill: only FP32 and FP16 are supported");
    if (device_.is_cuda() && value == 0.0f) {
        DeviceGuard g(device_);
        hip_check(hipMemset(data_, 0, nbytes_), "hipMemset");
        return;
    }
    Tensor host(shape_, dtype_, Device::cpu());
    if (dtype_ == DType::FP32) {
        auto* p = static_cast<float*>(host.data());
        for (int64_t i = 0; i < numel_; ++i) p[i] = value;
    } else {
        const uint16_t bits = half_bits(value);
        auto* p = static_cast<uint16_t*>(host.data());
        for (int64_t i = 0; i < numel_; ++i) p[i] = bits;
    }
    copy_raw(host.data(), data_, nbytes_, Device::cpu(), device_);
}

}  // namespace mini_infer
