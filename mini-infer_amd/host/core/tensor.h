// tensor.h -- the owning n-d buffer every layer signature uses.
//
// Same interface as the reference's mini_infer::Tensor (src/core/tensor.h:11-115)
// so layer code and callers compile unchanged: DType / Device / dtype_size /
// dtype_name, owning construction, deep copy, move, host<->device transfer,
// fill and contiguity.  `Device::cuda(i)` / `DeviceType::CUDA` keep the
// reference's names and denote GPU i of this HIP build; memory comes from
// hipMalloc.  Errors throw std::runtime_error.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

namespace mini_infer {

enum class DType : uint8_t {
    FP32 = 0,
    FP16 = 1,
    BF16 = 2,
    INT32 = 3,
    INT64 = 4,
};

enum class DeviceType : uint8_t {
    CPU = 0,
    CUDA = 1,  // the GPU (HIP device) -- name kept for source compatibility
};

struct Device {
    DeviceType type = DeviceType::CPU;
    int index = 0;

    bool is_cuda() const { return type == DeviceType::CUDA; }
    bool is_cpu() const { return type == DeviceType::CPU; }

    static Device cpu() { return {DeviceType::CPU, 0}; }
    static Device cuda(int idx = 0) { return {DeviceType::CUDA, idx}; }
};

inline std::size_t dtype_size(DType d) {
    switch (d) {
        case DType::FP32: return 4;
        case DType::FP16: return 2;
        case DType::BF16: return 2;
        case DType::INT32: return 4;
        case DType::INT64: return 8;
    }
    return 0;
}

const char* dtype_name(DType d);

class Tensor {
public:
    Tensor();
    Tensor(std::vector<int64_t> shape, DType dtype, Device device);

    static Tensor empty(std::vector<int64_t> shape, DType dtype, Device device);

    Tensor(const Tensor& other);             // deep copy
    Tensor& operator=(const Tensor& other);  // deep copy
    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(Tensor&& other) noexcept;
    ~Tensor();

    const std::vector<int64_t>& shape() const { return shape_; }
    const std::vector<int64_t>& stride() const { return stride_; }
    int64_t numel() const { return numel_; }
    std::size_t nbytes() const { return nbytes_; }
    DType dtype() const { return dtype_; }
    Device device() const { return device_; }
    int ndim() const { return static_cast<int>(shape_.size()); }
    void* data() { return data_; }
    const void* data() const { return data_; }
    bool owns_data() const { return owns_data_; }

    // Copy to another device (CPU <-> GPU, GPU <-> GPU); returns a new tensor.
    Tensor to(Device target) const;

    // Copy `bytes` between two buffers on the given devices (synchronous).
    static void copy_raw(const void* src, void* dst, std::size_t bytes, Device src_dev,
                         Device dst_dev);

    // Fill every element with `value` (FP32 / FP16, CPU or GPU).
    void fill(float value);

    bool is_contiguous() const;

private:
    void allocate_();
    void release_();
    void swap_(Tensor& other) noexcept;
    void compute_default_stride_();

    std::vector<int64_t> shape_;
    std::vector<int64_t> stride_;
    int64_t numel_ = 0;
    std::size_t nbytes_ = 0;
    DType dtype_ = DType::FP32;
    Device device_ = Device::cpu();
    void* data_ = nullptr;
    bool owns_data_ = false;
};

}  // namespace mini_infer
