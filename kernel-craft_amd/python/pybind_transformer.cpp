// pybind_transformer.cpp -- the `kernel_craft_transformer` Python module for
// the MI355X build of kernel-craft's quantization path.
//
// It registers the reference module's functions under the same names,
// argument names and defaults (pybind_transformer.cpp:801-882 in the
// reference): numpy arrays in, numpy arrays out; each call copies its
// inputs to the GPU, runs the library's C launcher on the null stream (the
// reference passes stream 0, :280,317,354) and copies the result back.
// Two functions the reference's docstring lists but never registers,
// `gemv_int4` and `smoothquant_scale` (:12,15), are registered here.
//
// Differences, each deliberate:
//  * inputs are converted to C-contiguous arrays of the expected dtype and
//    their sizes are checked against rows/cols (ValueError); the reference
//    reads whatever buffer it is given;
//  * a launcher that reports an error (kc_get_last_error) raises
//    RuntimeError with the library's message; a failed HIP call too;
//  * `rmsnorm` (:759-800,873) runs the library's launch_rmsnorm;
//  * the functions outside this path (attention, speculative decoding,
//    collectives, Mamba) are registered under their names and raise
//    NotImplementedError, as the library's C stubs report
//    KC_ERR_NOT_IMPLEMENTED.
#include <hip/hip_runtime_api.h>
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>

#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "kernel_craft.h"

namespace py = pybind11;

namespace {

template <typename T>
using carray = py::array_t<T, py::array::c_style | py::array::forcecast>;

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// A device allocation that frees itself.
class DeviceBuffer {
  public:
    explicit DeviceBuffer(size_t bytes) {
        if (bytes > 0) hip_check(hipMalloc(&p_, bytes), "hipMalloc");
    }
    ~DeviceBuffer() {
        if (p_) (void)hipFree(p_);
    }
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_) { o.p_ = nullptr; }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    template <typename T>
    T* as() const { return static_cast<T*>(p_); }

  private:
    void* p_ = nullptr;
};

template <typename T>
DeviceBuffer upload(const carray<T>& a) {
    const size_t bytes = static_cast<size_t>(a.size()) * sizeof(T);
    DeviceBuffer d(bytes);
    if (bytes) hip_check(hipMemcpy(d.as<void>(), a.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    return d;
}

template <typename T>
py::array_t<T> download(const DeviceBuffer& d, std::vector<py::ssize_t> shape) {
    py::array_t<T> out(shape);
    const size_t bytes = static_cast<size_t>(out.size()) * sizeof(T);
    if (bytes) hip_check(hipMemcpy(out.mutable_data(), d.as<void>(), bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return out;
}

// The launchers validate their arguments and record failures instead of
// returning them (their signatures are the reference's void ones).
void check_library(const char* name) {
    if (kc_get_last_error() != KC_SUCCESS) throw std::runtime_error(std::string(name) + ": " + kc_last_error_string());
}

void need(bool ok, const std::string& msg) {
    if (!ok) throw py::value_error(msg);
}

void check_int4(const char* fn, const carray<uint8_t>& packed, const carray<float>& scales,
                const carray<uint8_t>& zeros, int rows, int cols, int group_size) {
    need(rows >= 0 && cols >= 0, std::string(fn) + ": negative shape");
    need(group_size > 0 && cols % 2 == 0 && cols % group_size == 0,
         std::string(fn) + ": cols must be even and a multiple of group_size");
    const int64_t G = cols / group_size;
    need(packed.size() >= int64_t{rows} * (cols / 2), std::string(fn) + ": packed holds fewer than rows*cols/2 bytes");
    need(scales.size() >= int64_t{rows} * G, std::string(fn) + ": scales holds fewer than rows*(cols/group_size) values");
    // the kernels read zero byte (g/2) of a row of stride floor(G/2)
    // (quant_int4.cu:93,152): the last row reaches byte (rows-1)*floor(G/2) + (G-1)/2
    const int64_t zneed = rows == 0 || G == 0 ? 0 : int64_t{rows - 1} * (G / 2) + (G - 1) / 2 + 1;
    need(zeros.size() >= zneed, std::string(fn) + ": zeros is too small for rows and groups");
}

py::array_t<float> quant_int4_dequant(const carray<uint8_t>& packed, const carray<float>& scales,
                                      const carray<uint8_t>& zeros, int rows, int cols,
                                      int group_size) {
    check_int4("quant_int4_dequant", packed, scales, zeros, rows, cols, group_size);
    DeviceBuffer dp = upload(packed), ds = upload(scales), dz = upload(zeros);
    DeviceBuffer out(static_cast<size_t>(rows) * cols * sizeof(float));
    kc_get_last_error();
    launch_dequantize_int4(dp.as<uint8_t>(), ds.as<float>(), dz.as<uint8_t>(), out.as<float>(), rows, cols,
                           group_size, nullptr);
    check_library("quant_int4_dequant");
    return download<float>(out, {rows, cols});
}

py::array_t<float> gemv_int4(const carray<uint8_t>& packed, const carray<float>& scales,
                             const carray<uint8_t>& zeros, const carray<float>& x, int rows, int cols,
                             int group_size) {
    check_int4("gemv_int4", packed, scales, zeros, rows, cols, group_size);
    need(x.size() >= cols, "gemv_int4: x holds fewer than cols values");
    DeviceBuffer dp = upload(packed), ds = upload(scales), dz = upload(zeros), dx = upload(x);
    DeviceBuffer y(static_cast<size_t>(rows) * sizeof(float));
    kc_get_last_error();
    launch_gemv_int4(dp.as<uint8_t>(), ds.as<float>(), dz.as<uint8_t>(), dx.as<float>(), y.as<float>(), rows,
                     cols, group_size, nullptr);
    check_library("gemv_int4");
    return download<float>(y, {rows});
}

py::tuple fp8_quantize(const carray<float>& input, bool per_token) {
    need(input.ndim() == 2, "fp8_quantize: input must be 2-D [rows, cols]");
    const int rows = static_cast<int>(input.shape(0)), cols = static_cast<int>(input.shape(1));
    const int nscales = per_token ? rows : 1;
    DeviceBuffer di = upload(input);
    DeviceBuffer dq(static_cast<size_t>(rows) * cols);
    DeviceBuffer ds(static_cast<size_t>(std::max(nscales, 1)) * sizeof(float));
    if (!per_token) {
        // The per-tensor scale is computed on the host, as the reference's
        // binding does (:308-315): absmax with fmax from 0 (NaN ignored),
        // then absmax / 448, or 1 for an all-zero tensor.
        float amax = 0.0f;
        const float* p = input.data();
        for (py::ssize_t i = 0; i < input.size(); ++i) amax = std::fmax(amax, std::fabs(p[i]));
        const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
        hip_check(hipMemcpy(ds.as<void>(), &scale, sizeof(float), hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    kc_get_last_error();
    launch_quantize_fp8(di.as<float>(), dq.as<int8_t>(), ds.as<float>(), rows, cols, per_token, nullptr);
    check_library("fp8_quantize");
    return py::make_tuple(download<int8_t>(dq, {rows, cols}), download<float>(ds, {nscales}));
}

py::array_t<float> fp8_dequantize(const carray<int8_t>& quantized, const carray<float>& scales, int rows,
                                  int cols, bool per_token) {
    need(rows >= 0 && cols >= 0, "fp8_dequantize: negative shape");
    need(quantized.size() >= int64_t{rows} * cols, "fp8_dequantize: quantized holds fewer than rows*cols codes");
    need(scales.size() >= (per_token ? rows : 1), "fp8_dequantize: too few scales");
    DeviceBuffer dq = upload(quantized), ds = upload(scales);
    DeviceBuffer out(static_cast<size_t>(rows) * cols * sizeof(float));
    kc_get_last_error();
    launch_dequantize_fp8(dq.as<int8_t>(), ds.as<float>(), out.as<float>(), rows, cols, per_token, nullptr);
    check_library("fp8_dequantize");
    return download<float>(out, {rows, cols});
}

py::array_t<float> smoothquant_scale(const carray<float>& input, const carray<float>& smooth_scales) {
    need(input.ndim() == 2, "smoothquant_scale: input must be 2-D [rows, cols]");
    const int rows = static_cast<int>(input.shape(0)), cols = static_cast<int>(input.shape(1));
    need(smooth_scales.size() >= cols, "smoothquant_scale: smooth_scales holds fewer than cols values");
    DeviceBuffer di = upload(input), ds = upload(smooth_scales);
    DeviceBuffer out(static_cast<size_t>(rows) * cols * sizeof(float));
    kc_get_last_error();
    launch_smoothquant_scale(di.as<float>(), ds.as<float>(), out.as<float>(), rows, cols, nullptr);
    check_library("smoothquant_scale");
    return download<float>(out, {rows, cols});
}

// pybind_transformer.cpp:759-800 of the reference: x fp32 [rows, D], g [D].
py::array_t<float> rmsnorm(const carray<float>& x, const carray<float>& g, float eps) {
    need(x.ndim() == 2, "rmsnorm: x must be 2-D [rows, D]");
    need(g.ndim() == 1, "rmsnorm: g must be 1-D [D]");
    const int rows = static_cast<int>(x.shape(0)), D = static_cast<int>(x.shape(1));
    need(g.shape(0) == D, "rmsnorm: g.shape[0] must equal D");
    DeviceBuffer dx = upload(x), dg = upload(g);
    DeviceBuffer dy(static_cast<size_t>(rows) * D * sizeof(float));
    kc_get_last_error();
    launch_rmsnorm(dx.as<float>(), dg.as<float>(), dy.as<float>(), rows, D, eps, nullptr);
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    check_library("rmsnorm");
    return download<float>(dy, {rows, D});
}

void register_not_implemented(py::module_& m, const char* name, const char* doc) {
    const std::string msg = std::string(name) + " is outside the MI355X build's quantization path";
    m.def(
        name,
        [msg](py::args, py::kwargs) -> py::object {
            PyErr_SetString(PyExc_NotImplementedError, msg.c_str());
            throw py::error_already_set();
        },
        doc);
}

}  // namespace

PYBIND11_MODULE(kernel_craft_transformer, m) {
    m.doc() = "kernel-craft quantized-inference kernels on MI355X (gfx950): INT4 dequant/GEMV, FP8 E4M3, SmoothQuant";

    m.def("quant_int4_dequant", &quant_int4_dequant, py::arg("packed"), py::arg("scales"), py::arg("zeros"),
          py::arg("rows"), py::arg("cols"), py::arg("group_size") = 128, "Dequantize INT4 packed weights to FP32");
    m.def("gemv_int4", &gemv_int4, py::arg("packed"), py::arg("scales"), py::arg("zeros"), py::arg("x"),
          py::arg("rows"), py::arg("cols"), py::arg("group_size") = 128,
          "y = W x with INT4 weights dequantized on the fly (fp32 x and y)");
    m.def("fp8_quantize", &fp8_quantize, py::arg("input"), py::arg("per_token") = true,
          "Quantize FP32 activations to FP8 E4M3; returns (quantized, scales)");
    m.def("fp8_dequantize", &fp8_dequantize, py::arg("quantized"), py::arg("scales"), py::arg("rows"),
          py::arg("cols"), py::arg("per_token") = true, "Dequantize FP8 E4M3 back to FP32");
    m.def("smoothquant_scale", &smoothquant_scale, py::arg("input"), py::arg("smooth_scales"),
          "SmoothQuant activation smoothing: input / smooth_scales (per column)");
    m.def("rmsnorm", &rmsnorm, py::arg("x"), py::arg("g"), py::arg("eps") = 1e-6f,
          "RMSNorm: y = g * x / sqrt(mean(x^2) + eps) per row (fp32)");

    register_not_implemented(m, "flash_attention", "Not implemented in this build");
    register_not_implemented(m, "paged_attention", "Not implemented in this build");
    register_not_implemented(m, "speculative_decode", "Not implemented in this build");
    register_not_implemented(m, "ring_allreduce", "Not implemented in this build");
    register_not_implemented(m, "allgather", "Not implemented in this build");
    register_not_implemented(m, "col_parallel_linear", "Not implemented in this build");
    register_not_implemented(m, "row_parallel_linear", "Not implemented in this build");
    register_not_implemented(m, "nccl_comm_init", "Not implemented in this build");
    register_not_implemented(m, "nccl_comm_destroy", "Not implemented in this build");
    register_not_implemented(m, "nccl_allreduce", "Not implemented in this build");
    register_not_implemented(m, "nccl_group_start", "Not implemented in this build");
    register_not_implemented(m, "nccl_group_end", "Not implemented in this build");
    register_not_implemented(m, "selective_scan", "Not implemented in this build");
    register_not_implemented(m, "depthwise_conv1d", "Not implemented in this build");
    m.attr("HAVE_NCCL") = false;
}
