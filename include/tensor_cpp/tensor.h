/*
 * tensor_cpp/tensor.h - the host tensor type the reference's KV-cache and
 * attention APIs exchange (reference tensor_cpp/include/tensor_cpp/tensor.h:61-155).
 *
 * Only the part the attention path uses: a float-only, row-major, owning
 * tensor with its shape.  view() reinterprets the shape; transpose() returns a
 * materialised copy, as the reference's does.
 */
#ifndef SA_AMD_TENSOR_CPP_TENSOR_H
#define SA_AMD_TENSOR_CPP_TENSOR_H

#include <cstddef>
#include <initializer_list>
#include <string>
#include <vector>

namespace tensor_cpp {

class Shape {
public:
    std::vector<size_t> dims;

    Shape() = default;
    Shape(const std::vector<size_t>& d) : dims(d) {}
    Shape(std::initializer_list<size_t> init) : dims(init) {}

    size_t ndim() const { return dims.size(); }
    size_t operator[](size_t i) const { return dims[i]; }
    size_t& operator[](size_t i) { return dims[i]; }
    size_t total() const;
    bool operator==(const Shape& o) const { return dims == o.dims; }
    bool operator!=(const Shape& o) const { return dims != o.dims; }
    std::string to_string() const;
};

class Tensor {
public:
    Tensor() = default;
    explicit Tensor(const Shape& shape);
    Tensor(const Shape& shape, float value);
    Tensor(const std::vector<float>& data, const Shape& shape);
    Tensor(std::vector<float>&& data, const Shape& shape) noexcept;

    const Shape& shape() const { return shape_; }
    size_t ndim() const { return shape_.ndim(); }
    size_t size() const { return data_.size(); }
    size_t total() const { return shape_.total(); }
    float* data() { return data_.data(); }
    const float* data() const { return data_.data(); }
    float& operator[](size_t i) { return data_[i]; }
    const float& operator[](size_t i) const { return data_[i]; }

    Tensor view(const Shape& new_shape) const;
    Tensor reshape(const Shape& new_shape) const { return view(new_shape); }
    Tensor transpose(size_t dim1, size_t dim2) const;
    Tensor contiguous() const { return *this; }
    void fill(float value);
    void zero() { fill(0.0f); }

private:
    std::vector<float> data_;
    Shape shape_;
};

using TensorF = Tensor;

}  // namespace tensor_cpp

#endif
