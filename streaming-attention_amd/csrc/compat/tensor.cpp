// The host tensor of the API mirror (reference tensor_cpp/include/tensor_cpp/tensor.h:61-155).
#include "tensor_cpp/tensor.h"

#include <algorithm>
#include <stdexcept>
#include <utility>

namespace tensor_cpp {

size_t Shape::total() const {
    if (dims.empty()) return 0;
    size_t t = 1;
    for (size_t d : dims) t *= d;
    return t;
}

std::string Shape::to_string() const {
    std::string s = "(";
    for (size_t i = 0; i < dims.size(); ++i) {
        if (i) s += ", ";
        s += std::to_string(dims[i]);
    }
    return s + ")";
}

Tensor::Tensor(const Shape& shape) : data_(shape.total(), 0.0f), shape_(shape) {}

Tensor::Tensor(const Shape& shape, float value) : data_(shape.total(), value), shape_(shape) {}

Tensor::Tensor(const std::vector<float>& data, const Shape& shape) : data_(data), shape_(shape) {
    if (data_.size() != shape_.total()) throw std::invalid_argument("data size does not match shape");
}

Tensor::Tensor(std::vector<float>&& data, const Shape& shape) noexcept
    : data_(std::move(data)), shape_(shape) {}

Tensor Tensor::view(const Shape& new_shape) const {
    if (new_shape.total() != data_.size())
        throw std::invalid_argument("view: element count mismatch " + shape_.to_string() + " -> " +
                                    new_shape.to_string());
    return Tensor(data_, new_shape);
}

Tensor Tensor::transpose(size_t d1, size_t d2) const {
    const size_t nd = shape_.ndim();
    if (d1 >= nd || d2 >= nd) throw std::out_of_range("transpose: dimension out of range");
    Shape out_shape = shape_;
    std::swap(out_shape.dims[d1], out_shape.dims[d2]);
    std::vector<size_t> in_stride(nd, 1), out_stride(nd, 1);
    for (size_t i = nd - 1; i > 0; --i) {
        in_stride[i - 1] = in_stride[i] * shape_[i];
        out_stride[i - 1] = out_stride[i] * out_shape[i];
    }
    std::vector<float> out(data_.size());
    std::vector<size_t> idx(nd, 0);
    for (size_t flat = 0; flat < data_.size(); ++flat) {
        size_t rem = flat, src = 0;
        for (size_t i = 0; i < nd; ++i) {
            idx[i] = rem / out_stride[i];
            rem %= out_stride[i];
        }
        std::swap(idx[d1], idx[d2]);
        for (size_t i = 0; i < nd; ++i) src += idx[i] * in_stride[i];
        out[flat] = data_[src];
    }
    return Tensor(std::move(out), out_shape);
}

void Tensor::fill(float value) { std::fill(data_.begin(), data_.end(), value); }

}  // namespace tensor_cpp
