// Ctools.h -- the host-framework types the dispatch layer is written against.
//
// The reference is a plugin of the CTorch framework and includes CTorch's
// Ctools.h / Tensor.h for `op`, `DeviceType`, `DType` and `Tensor`
// (CMakeLists.txt:7-14); those headers are not part of the reference
// repository.  This file supplies the subset the hot path needs, with the
// same names, so the registry / hot-path manager / backward capture keep the
// reference's signatures.  Tensors here may live in HIP device memory
// (DeviceType::kHIP), which is how a registry hit reaches the GPU kernels.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace ct {

// Operator codes.  Order follows the prime codes of RollingHash::getOpCode
// (src/C3/RollingHash.cpp:44-70), which enumerate the host framework's ops.
enum class op : int {
    Add = 0, Sub, Neg, Mul, Div, MatMul, Dot, Cos, Sin, ReLU, Tanh, Sigmoid, GELU, LReLU, Log, Exp, Abs,
    Softmax, Min, Max, MSE, CE, MAE, Conv, Pool, kCount
};

// kHIP is the device this backend adds (the reference gates on kCPU,
// include/C3/C3HotPathManager.h:1007, src/C3/C3BackwardCapture.cpp:138-146).
enum class DeviceType : int { kCPU = 0, kCUDA = 1, kMPS = 2, kHIP = 3 };

enum class DType : int { kFloat = 0, kBFloat16 = 1 };

inline size_t dtypeSize(DType t) { return t == DType::kBFloat16 ? 2 : 4; }

struct ShapeTag {};

// Reference-counted buffer.  kHIP buffers come from a per-process caching
// pool (hipMalloc on a miss, never returned to the driver until
// releaseCachedDeviceMemory()) and belong to the stream that was current on
// the allocating thread: the pool hands a freed block to another stream only
// after that stream has been made to wait for the block's stream (see
// Ctools.cpp).  kCPU buffers are plain heap memory.  A borrowed buffer
// (fromBlob) is never freed.
class Storage {
public:
    Storage(size_t nbytes, DeviceType dev);
    Storage(void* borrowed, size_t nbytes, DeviceType dev) : ptr_(borrowed), nbytes_(nbytes), dev_(dev), owned_(false) {}
    ~Storage();
    Storage(const Storage&) = delete;
    Storage& operator=(const Storage&) = delete;
    void* data() const { return ptr_; }
    size_t nbytes() const { return nbytes_; }
    DeviceType device() const { return dev_; }

private:
    void* ptr_ = nullptr;
    size_t nbytes_ = 0;
    size_t capacity_ = 0;
    DeviceType dev_ = DeviceType::kCPU;
    bool owned_ = true;
    void* stream_ = nullptr;  // kHIP: stream current at allocation (hipStream_t)
};

// Free the HIP blocks held by the caching pool (called by shutdownAll).
void releaseCachedDeviceMemory();

class Tensor {
public:
    Tensor() = default;
    Tensor(ShapeTag, std::vector<size_t> shape, DType dt = DType::kFloat, DeviceType dev = DeviceType::kCPU);
    static Tensor fromBlob(void* data, std::vector<size_t> shape, DType dt, DeviceType dev);

    bool defined() const { return defined_; }
    const std::vector<size_t>& shape() const { return shape_; }
    const std::vector<size_t>& sizes() const { return shape_; }
    DeviceType device() const { return dev_; }
    DType dtype() const { return dtype_; }
    size_t numel() const;
    size_t nbytes() const { return numel() * dtypeSize(dtype_); }
    void* data() const { return storage_ ? storage_->data() : nullptr; }
    template <typename T>
    T* data_ptr() const { return static_cast<T*>(data()); }

private:
    std::shared_ptr<Storage> storage_;
    std::vector<size_t> shape_;
    DType dtype_ = DType::kFloat;
    DeviceType dev_ = DeviceType::kCPU;
    bool defined_ = false;
};

// Host-side diagnostics (CtorchError::log in the reference).
enum class ErrorLevel { DEBUG, INFO, WARN, ERROR };
void c3log(ErrorLevel lvl, const std::string& msg);

}  // namespace ct
