// tensor.h — device tensor of the qwen-image hot path on the HIP runtime.
//
// Same surface as the reference's Tensor / DType (qwen-image.cu tensor.h:39-238):
// an owning or non-owning pointer to device memory with up to five dims,
// alloc / alloc_like / zero / from_host / to_host / view / slice / clone,
// move-only. DType gains FP16 (the SageAttention inputs) and FP8_E4M3 (the
// e4m3 weight and activation bytes of QuantMode::FP8_HADAMARD).
//
// Errors behave as in the reference (tensor.h:15-37): a failing HIP call
// prints "HIP error at file:line: message" and exits with status 1.
#pragma once

#include <hip/hip_runtime.h>

#include <cassert>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <string>
#include <vector>

#define HIP_CHECK(call)                                                                      \
    do {                                                                                     \
        hipError_t err_ = (call);                                                            \
        if (err_ != hipSuccess) {                                                            \
            fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(err_)); \
            exit(1);                                                                         \
        }                                                                                    \
    } while (0)

enum class DType { BF16, FP32, INT8, INT32, UINT8, FP16, FP8_E4M3 };

inline size_t dtype_size(DType dt) {
    switch (dt) {
        case DType::BF16: return 2;
        case DType::FP32: return 4;
        case DType::INT8: return 1;
        case DType::INT32: return 4;
        case DType::UINT8: return 1;
        case DType::FP16: return 2;
        case DType::FP8_E4M3: return 1;
    }
    return 0;
}

inline const char* dtype_name(DType dt) {
    switch (dt) {
        case DType::BF16: return "BF16";
        case DType::FP32: return "FP32";
        case DType::INT8: return "INT8";
        case DType::INT32: return "INT32";
        case DType::UINT8: return "UINT8";
        case DType::FP16: return "FP16";
        case DType::FP8_E4M3: return "FP8_E4M3";
    }
    return "???";
}

struct Tensor {
    void* data = nullptr;
    int64_t shape[5] = {0, 0, 0, 0, 0};
    int ndim = 0;
    DType dtype = DType::BF16;
    bool owns_data = false;

    Tensor() = default;
    Tensor(const Tensor&) = delete;
    Tensor& operator=(const Tensor&) = delete;

    Tensor(Tensor&& o) noexcept { take(o); }
    Tensor& operator=(Tensor&& o) noexcept {
        if (this != &o) {
            free_data();
            take(o);
        }
        return *this;
    }
    ~Tensor() { free_data(); }

    void free_data() {
        if (data && owns_data) HIP_CHECK(hipFree(data));
        data = nullptr;
        owns_data = false;
    }

    int64_t numel() const {
        if (ndim == 0) return 0;
        int64_t n = 1;
        for (int i = 0; i < ndim; ++i) n *= shape[i];
        return n;
    }

    size_t nbytes() const { return static_cast<size_t>(numel()) * dtype_size(dtype); }

    static Tensor alloc(std::initializer_list<int64_t> dims, DType dt = DType::BF16) {
        return alloc(std::vector<int64_t>(dims), dt);
    }

    static Tensor alloc(const std::vector<int64_t>& dims, DType dt = DType::BF16) {
        Tensor t;
        t.set_shape(dims);
        t.dtype = dt;
        t.owns_data = true;
        if (t.nbytes() > 0) HIP_CHECK(hipMalloc(&t.data, t.nbytes()));
        return t;
    }

    static Tensor alloc_like(const Tensor& o) {
        return alloc(std::vector<int64_t>(o.shape, o.shape + o.ndim), o.dtype);
    }

    // Non-owning tensor over existing device memory.
    static Tensor wrap(void* ptr, const std::vector<int64_t>& dims, DType dt) {
        Tensor t;
        t.data = ptr;
        t.set_shape(dims);
        t.dtype = dt;
        return t;
    }

    void zero() {
        if (nbytes()) HIP_CHECK(hipMemset(data, 0, nbytes()));
    }

    void from_host(const void* host, size_t bytes) {
        assert(bytes <= nbytes());
        HIP_CHECK(hipMemcpy(data, host, bytes, hipMemcpyHostToDevice));
    }
    void from_host(const void* host) { from_host(host, nbytes()); }

    void to_host(void* host, size_t bytes) const {
        assert(bytes <= nbytes());
        HIP_CHECK(hipMemcpy(host, data, bytes, hipMemcpyDeviceToHost));
    }
    void to_host(void* host) const { to_host(host, nbytes()); }

    Tensor view(std::initializer_list<int64_t> dims) const { return view(std::vector<int64_t>(dims)); }
    Tensor view(const std::vector<int64_t>& dims) const {
        Tensor t = wrap(data, dims, dtype);
        assert(t.numel() == numel());
        return t;
    }

    // Non-owning view of rows [start, end) along dimension 0.
    Tensor slice(int64_t start, int64_t end) const {
        assert(ndim >= 1 && start >= 0 && end <= shape[0] && start < end);
        int64_t inner = 1;
        for (int i = 1; i < ndim; ++i) inner *= shape[i];
        std::vector<int64_t> dims(shape, shape + ndim);
        dims[0] = end - start;
        return wrap(static_cast<char*>(data) + start * inner * dtype_size(dtype), dims, dtype);
    }

    Tensor clone() const {
        Tensor t = alloc_like(*this);
        if (nbytes()) HIP_CHECK(hipMemcpy(t.data, data, nbytes(), hipMemcpyDeviceToDevice));
        return t;
    }

    std::string shape_str() const {
        std::string s = "[";
        for (int i = 0; i < ndim; ++i) {
            if (i) s += ", ";
            s += std::to_string(shape[i]);
        }
        return s + "]";
    }

    void print_info(const char* name = "") const {
        fprintf(stderr, "Tensor %s: %s %s, %zu bytes\n", name, shape_str().c_str(), dtype_name(dtype), nbytes());
    }

  private:
    void set_shape(const std::vector<int64_t>& dims) {
        assert(dims.size() <= 5);
        ndim = static_cast<int>(dims.size());
        for (int i = 0; i < 5; ++i) shape[i] = i < ndim ? dims[i] : 0;
    }
    void take(Tensor& o) {
        data = o.data;
        memcpy(shape, o.shape, sizeof(shape));
        ndim = o.ndim;
        dtype = o.dtype;
        owns_data = o.owns_data;
        o.data = nullptr;
        o.owns_data = false;
    }
};
