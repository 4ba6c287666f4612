/*
 * tensor_cpp/tensor.h - the host tensor the reference's API exchanges
 * (reference tensor_cpp/include/tensor_cpp/tensor.h:16-155).
 *
 * A float-only, row-major, owning tensor with its shape, with the reference's
 * members: element access, element-wise arithmetic, reductions, matmul,
 * transposes, reshapes, element-wise math, fills and factories.  Tensors live
 * in host memory as there; element-wise operations and reductions are host
 * loops over that memory, as the reference's are, and matmul runs on the GPU
 * (fp32 MFMA).  view() and reshape() reinterpret the shape of a copy;
 * transpose() returns a materialised copy.
 */
#ifndef SA_AMD_TENSOR_CPP_TENSOR_H
#define SA_AMD_TENSOR_CPP_TENSOR_H

#include <cstddef>
#include <initializer_list>
#include <iomanip>
#include <iostream>
#include <memory>
#include <stdexcept>
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
    Tensor(const Tensor& other) = default;
    Tensor(Tensor&& other) noexcept = default;
    Tensor& operator=(const Tensor& other) = default;
    Tensor& operator=(Tensor&& other) noexcept = default;

    const Shape& shape() const { return shape_; }
    size_t ndim() const { return shape_.ndim(); }
    size_t size() const { return data_.size(); }
    size_t total() const { return shape_.total(); }
    float* data() { return data_.data(); }
    const float* data() const { return data_.data(); }
    float& operator[](size_t i) { return data_[i]; }
    const float& operator[](size_t i) const { return data_[i]; }
    /* Element at a full row-major index. */
    float& operator()(const std::vector<size_t>& indices);
    const float& operator()(const std::vector<size_t>& indices) const;

    /* Element-wise, same shapes (std::invalid_argument otherwise). */
    Tensor operator+(const Tensor& other) const;
    Tensor operator+(float scalar) const;
    Tensor operator-(const Tensor& other) const;
    Tensor operator*(const Tensor& other) const;
    Tensor operator*(float scalar) const;
    Tensor operator/(const Tensor& other) const;
    Tensor operator/(float scalar) const;
    Tensor& operator+=(const Tensor& other);
    Tensor& operator*=(float scalar);

    float sum() const;
    float mean() const;
    float max() const;   // std::runtime_error when empty
    float min() const;

    /* [M, K] x [K, N] -> [M, N], on the GPU. */
    Tensor matmul(const Tensor& other) const;
    Tensor transpose() const;                       // 2-D
    Tensor transpose(size_t dim1, size_t dim2) const;

    Tensor reshape(const Shape& new_shape) const;   // same element count
    Tensor view(const Shape& new_shape) const { return reshape(new_shape); }
    Tensor contiguous() const { return *this; }
    Tensor squeeze() const;                         // drops every size-1 dim (keeps one)
    Tensor unsqueeze(size_t dim) const;

    Tensor exp() const;
    Tensor log() const;
    Tensor sqrt() const;
    Tensor square() const;
    Tensor abs() const;

    void fill(float value);
    void zero() { fill(0.0f); }
    std::string to_string() const;

    static Tensor zeros(const Shape& shape);
    static Tensor ones(const Shape& shape);
    static Tensor randn(const Shape& shape);
    static Tensor uniform(const Shape& shape, float low = 0, float high = 1);
    static Tensor eye(size_t n, size_t m = 0);

private:
    std::vector<float> data_;
    Shape shape_;
};

using TensorF = Tensor;

}  // namespace tensor_cpp

#endif
