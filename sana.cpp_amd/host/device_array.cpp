#include "device_array.h"

#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <stdexcept>
#include <string>

#include "../../include/sana_dit.h"

namespace sana_host {
namespace {

void hip_ok(hipError_t e, const char * what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void select_device() {
    thread_local bool done = false;
    if (done) return;
    const char * e = std::getenv("SANA_HIP_DEVICE");
    hip_ok(hipSetDevice(e ? std::atoi(e) : 0), "hipSetDevice");
    done = true;
}

}  // namespace

DeviceArray::DeviceArray(size_t n) : n_(n) {
    select_device();
    hip_ok(hipMalloc(reinterpret_cast<void **>(&p_), (n ? n : 1) * sizeof(float)), "hipMalloc");
}

DeviceArray::DeviceArray(const float * host, size_t n) : DeviceArray(n) {
    if (n) hip_ok(hipMemcpy(p_, host, n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy H2D");
}

DeviceArray::DeviceArray(const Tensor & t) : DeviceArray(t.data().data(), t.numel()) {}

DeviceArray::~DeviceArray() {
    if (p_) (void)hipFree(p_);
}

DeviceArray::DeviceArray(DeviceArray && o) noexcept : p_(o.p_), n_(o.n_) {
    o.p_ = nullptr;
    o.n_ = 0;
}

DeviceArray & DeviceArray::operator=(DeviceArray && o) noexcept {
    if (this != &o) {
        if (p_) (void)hipFree(p_);
        p_ = o.p_;
        n_ = o.n_;
        o.p_ = nullptr;
        o.n_ = 0;
    }
    return *this;
}

void DeviceArray::download(float * host, size_t n) const {
    if (n > n_) throw std::runtime_error("download larger than the device array");
    hip_ok(hipDeviceSynchronize(), "device work");
    if (n) hip_ok(hipMemcpy(host, p_, n * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

Tensor DeviceArray::to_tensor(std::vector<size_t> shape) const {
    Tensor t(std::move(shape));
    download(t.data().data(), t.numel());
    return t;
}

float * opt(const DeviceArray * a) { return a ? a->get() : nullptr; }

void op_check(int rc) {
    if (rc == SANA_OK) return;
    const std::string msg = sana_dit_last_error();
    if (rc == SANA_ERR_INVALID_ARGUMENT || rc == SANA_ERR_SHAPE) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

}  // namespace sana_host
