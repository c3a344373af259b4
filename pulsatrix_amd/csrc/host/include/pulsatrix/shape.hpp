/** @file shape.hpp
 *  @brief Tensor shape: dims, rank, numel (the surface of include/pulsatrix/shape.hpp).
 */
#pragma once

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <stdexcept>
#include <string>
#include <vector>

namespace pulsatrix {

class Shape {
public:
    Shape() = default;
    Shape(std::initializer_list<int64_t> dims) : dims_(dims) { validate(); }
    explicit Shape(std::vector<int64_t> dims) : dims_(std::move(dims)) { validate(); }

    [[nodiscard]] int64_t rank() const noexcept { return static_cast<int64_t>(dims_.size()); }
    [[nodiscard]] int64_t dim(size_t i) const {
        if (i >= dims_.size()) throw std::out_of_range("Shape::dim: axis out of range");
        return dims_[i];
    }
    [[nodiscard]] int64_t numel() const noexcept {
        if (dims_.empty()) return 0;
        int64_t n = 1;
        for (int64_t d : dims_) n *= d;
        return n;
    }
    [[nodiscard]] const std::vector<int64_t>& dims() const noexcept { return dims_; }
    bool operator==(const Shape& o) const noexcept { return dims_ == o.dims_; }
    bool operator!=(const Shape& o) const noexcept { return dims_ != o.dims_; }
    [[nodiscard]] std::string to_string() const {
        std::string s = "(";
        for (size_t i = 0; i < dims_.size(); ++i) s += (i ? ", " : "") + std::to_string(dims_[i]);
        return s + ")";
    }

private:
    void validate() const {
        for (int64_t d : dims_)
            if (d < 0) throw std::invalid_argument("Shape: dimensions must be non-negative");
    }
    std::vector<int64_t> dims_;
};

}  // namespace pulsatrix
