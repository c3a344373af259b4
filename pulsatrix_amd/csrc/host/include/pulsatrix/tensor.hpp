/** @file tensor.hpp
 *  @brief fp32 device tensor owning a buffer allocated through a DeviceBackend (the surface of
 *         include/pulsatrix/tensor.hpp:29-275).
 *
 *  As in the reference, every public constructor zero-fills or uploads (tensor.cpp:24-58) and a
 *  copy is a deep device-to-device copy (tensor.cpp:133-146). Tensor::uninitialized() is the
 *  addition the fused module path uses for buffers it overwrites completely.
 */
#pragma once

#include <initializer_list>
#include <vector>

#include "pulsatrix/device_backend.hpp"
#include "pulsatrix/shape.hpp"

namespace pulsatrix {

class Tensor {
public:
    Tensor() = default;
    Tensor(Shape shape, DeviceBackend* backend);
    Tensor(Shape shape, DeviceBackend* backend, DeviceType device);
    Tensor(Shape shape, DeviceBackend* backend, std::initializer_list<float> values, DeviceType device);
    Tensor(Shape shape, DeviceBackend* backend, std::initializer_list<float> values);
    Tensor(Shape shape, DeviceBackend* backend, const std::vector<float>& values, DeviceType device);
    Tensor(Shape shape, DeviceBackend* backend, const std::vector<float>& values);
    ~Tensor();

    /** @brief A tensor whose contents are undefined until written (no fill kernel). */
    static Tensor uninitialized(Shape shape, DeviceBackend* backend);

    Tensor(const Tensor& other);
    Tensor& operator=(const Tensor& other);
    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(Tensor&& other) noexcept;

    [[nodiscard]] const Shape& shape() const noexcept { return shape_; }
    [[nodiscard]] int64_t numel() const noexcept { return shape_.numel(); }
    [[nodiscard]] int64_t rank() const noexcept { return shape_.rank(); }
    [[nodiscard]] float* data() noexcept { return data_; }
    [[nodiscard]] const float* data() const noexcept { return data_; }
    [[nodiscard]] DeviceBackend* backend() const noexcept { return backend_; }
    [[nodiscard]] DeviceType device() const noexcept { return device_; }
    [[nodiscard]] bool requires_grad() const noexcept { return requires_grad_; }
    void set_requires_grad(bool r) noexcept { requires_grad_ = r; }

    /** @brief Metadata-only reshape; the element count must not change. */
    void reshape(Shape shape);
    [[nodiscard]] std::vector<float> to_host_vector() const;
    void fill(float value);
    /** @brief this += other (same shape). */
    void accumulate(const Tensor& other);

private:
    void allocate_storage();
    void release() noexcept;

    Shape shape_;
    DeviceBackend* backend_ = nullptr;
    DeviceType device_ = DeviceType::Cpu;
    float* data_ = nullptr;
    bool requires_grad_ = true;
};

/** @brief Throws std::invalid_argument unless t lives on `device` (tensor.hpp:285-301). */
void require_device(const Tensor& t, DeviceType device, const char* where);

}  // namespace pulsatrix
