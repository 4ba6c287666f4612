// The host tensor of the API mirror (reference tensor_cpp/include/tensor_cpp/tensor.h:16-155,
// tensor_cpp/src/tensor.cpp).  Element-wise work is a host loop over host
// memory, as in the reference; matmul runs on the GPU's fp32 linear kernel.
#include "tensor_cpp/tensor.h"

#include <algorithm>
#include <cmath>
#include <numeric>
#include <random>
#include <sstream>
#include <stdexcept>
#include <utility>

#include "device.h"

namespace tensor_cpp {

namespace {

// out[i] = f(a[i], b[i]) over two tensors of one shape.
template <class F>
Tensor zip(const Tensor& a, const Tensor& b, const char* what, F f) {
    if (a.shape() != b.shape()) throw std::invalid_argument(std::string("Shape mismatch for ") + what);
    std::vector<float> out(a.size());
    for (size_t i = 0; i < out.size(); ++i) out[i] = f(a[i], b[i]);
    return Tensor(std::move(out), a.shape());
}

template <class F>
Tensor map(const Tensor& a, F f) {
    std::vector<float> out(a.size());
    for (size_t i = 0; i < out.size(); ++i) out[i] = f(a[i]);
    return Tensor(std::move(out), a.shape());
}

}  // namespace

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

float& Tensor::operator()(const std::vector<size_t>& idx) {
    return const_cast<float&>(static_cast<const Tensor&>(*this)(idx));
}

const float& Tensor::operator()(const std::vector<size_t>& idx) const {
    if (idx.size() != shape_.ndim()) throw std::invalid_argument("index rank does not match the tensor");
    size_t flat = 0;
    for (size_t d = 0; d < idx.size(); ++d) {
        if (idx[d] >= shape_[d]) throw std::out_of_range("index out of range");
        flat = flat * shape_[d] + idx[d];
    }
    return data_[flat];
}

Tensor Tensor::operator+(const Tensor& o) const { return zip(*this, o, "addition", [](float a, float b) { return a + b; }); }
Tensor Tensor::operator-(const Tensor& o) const { return zip(*this, o, "subtraction", [](float a, float b) { return a - b; }); }
Tensor Tensor::operator*(const Tensor& o) const { return zip(*this, o, "multiplication", [](float a, float b) { return a * b; }); }
Tensor Tensor::operator/(const Tensor& o) const { return zip(*this, o, "division", [](float a, float b) { return a / b; }); }
Tensor Tensor::operator+(float s) const { return map(*this, [s](float a) { return a + s; }); }
Tensor Tensor::operator*(float s) const { return map(*this, [s](float a) { return a * s; }); }
Tensor Tensor::operator/(float s) const { return map(*this, [s](float a) { return a / s; }); }

Tensor& Tensor::operator+=(const Tensor& o) {
    if (shape_ != o.shape_) throw std::invalid_argument("Shape mismatch for in-place addition");
    for (size_t i = 0; i < data_.size(); ++i) data_[i] += o.data_[i];
    return *this;
}

Tensor& Tensor::operator*=(float s) {
    for (float& x : data_) x *= s;
    return *this;
}

float Tensor::sum() const { return std::accumulate(data_.begin(), data_.end(), 0.0f); }

float Tensor::mean() const { return data_.empty() ? 0.0f : sum() / static_cast<float>(data_.size()); }

float Tensor::max() const {
    if (data_.empty()) throw std::runtime_error("Cannot compute max of empty tensor");
    return *std::max_element(data_.begin(), data_.end());
}

float Tensor::min() const {
    if (data_.empty()) throw std::runtime_error("Cannot compute min of empty tensor");
    return *std::min_element(data_.begin(), data_.end());
}

Tensor Tensor::matmul(const Tensor& other) const {
    if (ndim() != 2 || other.ndim() != 2) throw std::invalid_argument("Matrix multiplication requires 2D tensors");
    if (shape_[1] != other.shape_[0]) throw std::invalid_argument("Shape mismatch for matrix multiplication");
    const size_t M = shape_[0], K = shape_[1], N = other.shape_[1];
    std::vector<float> out(M * N, 0.0f);
    if (M && N) {
        if (M > 0x7fffffffu || K > 0x7fffffffu || N > 0x7fffffffu)
            throw std::invalid_argument("matmul dimensions exceed the kernels' int range");
        // y = x . W^T with W = other^T [N][K]
        const Tensor wt = other.transpose();
        auto& st = sa_compat::staging();
        float* dx = st.in[0].as<float>(M * K);
        float* dw = st.in[1].as<float>(N * K);
        float* dy = st.out.as<float>(M * N);
        sa_compat::to_device(dx, data_.data(), M * K * sizeof(float));
        sa_compat::to_device(dw, wt.data(), N * K * sizeof(float));
        sa_compat::check(sa_linear_f32(dx, (int)M, (int)K, dw, (int)N, nullptr, dy, nullptr), "sa_linear_f32");
        sa_compat::to_host(out.data(), dy, M * N * sizeof(float));
    }
    return Tensor(std::move(out), Shape({M, N}));
}

Tensor Tensor::transpose() const {
    if (ndim() != 2) throw std::invalid_argument("Transpose only supports 2D tensors");
    return transpose(0, 1);
}

Tensor Tensor::transpose(size_t d1, size_t d2) const {
    const size_t nd = shape_.ndim();
    if (d1 >= nd || d2 >= nd) throw std::out_of_range("Dimension index out of range");
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

Tensor Tensor::reshape(const Shape& new_shape) const {
    if (new_shape.total() != data_.size())
        throw std::invalid_argument("New shape must have same total size: " + shape_.to_string() + " -> " +
                                    new_shape.to_string());
    return Tensor(data_, new_shape);
}

Tensor Tensor::squeeze() const {
    std::vector<size_t> dims;
    for (size_t d : shape_.dims)
        if (d != 1) dims.push_back(d);
    if (dims.empty()) dims.push_back(1);
    return reshape(Shape(dims));
}

Tensor Tensor::unsqueeze(size_t dim) const {
    if (dim > shape_.ndim()) throw std::out_of_range("unsqueeze: dimension out of range");
    std::vector<size_t> dims = shape_.dims;
    dims.insert(dims.begin() + static_cast<long>(dim), 1);
    return reshape(Shape(dims));
}

Tensor Tensor::exp() const { return map(*this, [](float a) { return std::exp(a); }); }
Tensor Tensor::log() const { return map(*this, [](float a) { return std::log(a); }); }
Tensor Tensor::sqrt() const { return map(*this, [](float a) { return std::sqrt(a); }); }
Tensor Tensor::square() const { return map(*this, [](float a) { return a * a; }); }
Tensor Tensor::abs() const { return map(*this, [](float a) { return std::fabs(a); }); }

void Tensor::fill(float value) { std::fill(data_.begin(), data_.end(), value); }

std::string Tensor::to_string() const {
    std::ostringstream os;
    os << "Tensor(shape=" << shape_.to_string() << ")\ndata:\n";
    if (data_.empty()) return os.str() + "  []\n";
    os << std::fixed << std::setprecision(4);
    if (ndim() == 1) {
        os << "  [";
        for (size_t i = 0; i < data_.size(); ++i) os << (i ? ", " : "") << data_[i];
        os << "]";
    } else if (ndim() == 2) {
        const size_t rows = shape_[0], cols = shape_[1];
        os << "  [[";
        for (size_t r = 0; r < rows; ++r) {
            if (r) os << "   [";
            for (size_t c = 0; c < cols; ++c) os << (c ? ", " : "") << data_[r * cols + c];
            os << "]" << (r + 1 < rows ? ",\n" : "");
        }
        os << "]";
    }
    return os.str();
}

Tensor Tensor::zeros(const Shape& shape) { return Tensor(shape, 0.0f); }
Tensor Tensor::ones(const Shape& shape) { return Tensor(shape, 1.0f); }

Tensor Tensor::randn(const Shape& shape) {
    Tensor t(shape);
    std::mt19937 gen(std::random_device{}());
    std::normal_distribution<float> dist(0.0f, 1.0f);
    for (float& x : t.data_) x = dist(gen);
    return t;
}

Tensor Tensor::uniform(const Shape& shape, float low, float high) {
    Tensor t(shape);
    std::mt19937 gen(std::random_device{}());
    std::uniform_real_distribution<float> dist(low, high);
    for (float& x : t.data_) x = dist(gen);
    return t;
}

Tensor Tensor::eye(size_t n, size_t m) {
    if (m == 0) m = n;
    Tensor t(Shape({n, m}), 0.0f);
    for (size_t i = 0; i < std::min(n, m); ++i) t.data_[i * m + i] = 1.0f;
    return t;
}

}  // namespace tensor_cpp
