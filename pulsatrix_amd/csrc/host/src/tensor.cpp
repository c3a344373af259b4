// Tensor: RAII fp32 buffer through a DeviceBackend (src/tensor.cpp semantics).
#include "pulsatrix/tensor.hpp"

#include <stdexcept>
#include <string>

namespace pulsatrix {

namespace {
CopyDirection upload_dir(DeviceType d) { return d == DeviceType::Cpu ? CopyDirection::HostToHost : CopyDirection::HostToDevice; }
CopyDirection download_dir(DeviceType d) {
    return d == DeviceType::Cpu ? CopyDirection::HostToHost : CopyDirection::DeviceToHost;
}
}  // namespace

void Tensor::allocate_storage() {
    if (backend_ == nullptr) throw std::invalid_argument("Tensor: backend must not be null");
    const int64_t n = shape_.numel();
    data_ = n > 0 ? static_cast<float*>(backend_->allocate(static_cast<size_t>(n) * sizeof(float))) : nullptr;
}

void Tensor::release() noexcept {
    if (backend_ && data_) backend_->free(data_);
    data_ = nullptr;
}

Tensor::Tensor(Shape shape, DeviceBackend* backend)
    : Tensor(std::move(shape), backend, backend ? backend->device() : DeviceType::Cpu) {}

Tensor::Tensor(Shape shape, DeviceBackend* backend, DeviceType device)
    : shape_(std::move(shape)), backend_(backend), device_(device) {
    allocate_storage();
    if (data_) backend_->fill(data_, 0.0f, static_cast<size_t>(numel()));  // zero-filled (tensor.cpp:24-30)
}

Tensor::Tensor(Shape shape, DeviceBackend* backend, const std::vector<float>& values, DeviceType device)
    : shape_(std::move(shape)), backend_(backend), device_(device) {
    if (static_cast<int64_t>(values.size()) != shape_.numel())
        throw std::invalid_argument("Tensor: " + std::to_string(values.size()) + " values for shape " +
                                    shape_.to_string());
    allocate_storage();
    if (data_) backend_->copy(data_, values.data(), values.size() * sizeof(float), upload_dir(device_));
}

Tensor::Tensor(Shape shape, DeviceBackend* backend, const std::vector<float>& values)
    : Tensor(std::move(shape), backend, values, backend ? backend->device() : DeviceType::Cpu) {}

Tensor::Tensor(Shape shape, DeviceBackend* backend, std::initializer_list<float> values, DeviceType device)
    : Tensor(std::move(shape), backend, std::vector<float>(values), device) {}

Tensor::Tensor(Shape shape, DeviceBackend* backend, std::initializer_list<float> values)
    : Tensor(std::move(shape), backend, std::vector<float>(values)) {}

Tensor Tensor::uninitialized(Shape shape, DeviceBackend* backend) {
    Tensor t;
    t.shape_ = std::move(shape);
    t.backend_ = backend;
    t.device_ = backend ? backend->device() : DeviceType::Cpu;
    t.allocate_storage();
    return t;
}

Tensor::~Tensor() { release(); }

Tensor::Tensor(const Tensor& other)
    : shape_(other.shape_), backend_(other.backend_), device_(other.device_), requires_grad_(other.requires_grad_) {
    if (backend_ == nullptr) return;
    allocate_storage();
    if (data_)
        backend_->copy(data_, other.data_, static_cast<size_t>(numel()) * sizeof(float),
                       device_ == DeviceType::Cpu ? CopyDirection::HostToHost : CopyDirection::DeviceToDevice);
}

Tensor& Tensor::operator=(const Tensor& other) {
    if (this == &other) return *this;
    Tensor tmp(other);
    *this = std::move(tmp);
    return *this;
}

Tensor::Tensor(Tensor&& other) noexcept
    : shape_(std::move(other.shape_)),
      backend_(other.backend_),
      device_(other.device_),
      data_(other.data_),
      requires_grad_(other.requires_grad_) {
    other.data_ = nullptr;
    other.shape_ = Shape();
}

Tensor& Tensor::operator=(Tensor&& other) noexcept {
    if (this == &other) return *this;
    release();
    shape_ = std::move(other.shape_);
    backend_ = other.backend_;
    device_ = other.device_;
    data_ = other.data_;
    requires_grad_ = other.requires_grad_;
    other.data_ = nullptr;
    other.shape_ = Shape();
    return *this;
}

void Tensor::reshape(Shape shape) {
    if (shape.numel() != shape_.numel())
        throw std::invalid_argument("Tensor::reshape: " + shape_.to_string() + " has a different element count than " +
                                    shape.to_string());
    shape_ = std::move(shape);
}

std::vector<float> Tensor::to_host_vector() const {
    std::vector<float> out(static_cast<size_t>(numel()));
    if (!out.empty()) backend_->copy(out.data(), data_, out.size() * sizeof(float), download_dir(device_));
    return out;
}

void Tensor::fill(float value) {
    if (data_) backend_->fill(data_, value, static_cast<size_t>(numel()));
}

void Tensor::accumulate(const Tensor& other) {
    if (other.shape_ != shape_) throw std::invalid_argument("Tensor::accumulate: shapes differ");
    if (data_) backend_->add(data_, other.data_, data_, static_cast<size_t>(numel()));
}

void require_device(const Tensor& t, DeviceType device, const char* where) {
    if (t.device() != device)
        throw std::invalid_argument(std::string(where) + ": tensor lives on a different device than the module");
}

}  // namespace pulsatrix
