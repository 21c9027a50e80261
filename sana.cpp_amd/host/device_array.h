// fp32 device arrays for the op-level API: HIP device memory on the device
// named by SANA_HIP_DEVICE (default 0), filled from and copied back to host
// memory synchronously.  Errors throw std::runtime_error; a failed op launcher
// (sana_op_*) throws the exception type its status code maps to.
#pragma once

#include <cstddef>
#include <vector>

#include "tensor.h"

namespace sana_host {

class DeviceArray {
public:
    explicit DeviceArray(size_t n);                 // uninitialised
    DeviceArray(const float * host, size_t n);      // copy of host[0, n)
    explicit DeviceArray(const Tensor & t);         // copy of the tensor's values
    ~DeviceArray();
    DeviceArray(DeviceArray && o) noexcept;
    DeviceArray & operator=(DeviceArray && o) noexcept;
    DeviceArray(const DeviceArray &) = delete;
    DeviceArray & operator=(const DeviceArray &) = delete;

    float * get() const { return p_; }
    size_t size() const { return n_; }
    void download(float * host, size_t n) const;    // waits for queued work first
    Tensor to_tensor(std::vector<size_t> shape) const;

private:
    float * p_ = nullptr;
    size_t n_ = 0;
};

// Device pointer of an optional tensor (null stays null).
float * opt(const DeviceArray * a);

// Throws for a non-zero sana_op_* / sana_dit_* status.
void op_check(int rc);

}  // namespace sana_host
