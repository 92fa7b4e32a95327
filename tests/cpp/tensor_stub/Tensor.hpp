// Tensor.hpp -- test stand-in for the caller-side Tensor that
// include/VedicGEMM.hpp works on.  Written for the tests of this repository:
// it has the members the GEMM surface uses (row-major float data, shape,
// total_size, rows() = shape[-2] or 1, cols() = shape[-1] or 0, checked at(),
// flat operator[], positive dimensions), which is the interface of LOGOS's
// include/Tensor.hpp:43-89.  Nothing else of that class is needed here.
#pragma once

#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

class Tensor {
public:
    std::vector<float> data;
    std::vector<int> shape;
    int total_size = 0;

    Tensor() = default;
    explicit Tensor(std::vector<int> dims, float fill = 0.0f) : shape(std::move(dims)) {
        long n = 1;
        for (int d : shape) {
            if (d <= 0) throw std::invalid_argument("Shape dimension must be > 0");
            n *= d;
        }
        total_size = (int)n;
        data.assign((size_t)n, fill);
    }

    int rows() const { return shape.size() >= 2 ? shape[shape.size() - 2] : 1; }
    int cols() const { return shape.empty() ? 0 : shape.back(); }

    float& at(int r, int c) { return data[index(r, c)]; }
    float at(int r, int c) const { return data[index(r, c)]; }
    float& operator[](int i) { return data[(size_t)i]; }
    float operator[](int i) const { return data[(size_t)i]; }

private:
    size_t index(int r, int c) const {
        if (r < 0 || c < 0 || r >= rows() || c >= cols())
            throw std::out_of_range("at(" + std::to_string(r) + "," + std::to_string(c) + ")");
        return (size_t)r * cols() + c;
    }
};
