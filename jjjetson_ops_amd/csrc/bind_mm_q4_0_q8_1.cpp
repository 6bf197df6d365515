// Python module `mm_q4_0_q8_1_me`: the reference's binding surface
// (src/bindings/mm_q4_0_q8_1_binding.cpp:12-23) over the C ABI of this library.
//   mmq(weight_q4_0: uint8, input: float32, quant_workspace: uint8, output: float32,
//       input_dims: list[int], nrows_out: int, ncols_k: int) -> None
// Writes quant_workspace (Q8_1 blocks, quantizer layout) and output (fp32,
// output[t*nrows_out + n]) in place.  Errors raise instead of printing.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <string>
#include <vector>

#include "jjjetson_ops_amd.h"

namespace py = pybind11;

namespace {

void check_contiguous(const py::array &a, const char *name) {
    const int f = a.flags();
    if (!(f & py::array::c_style) && !(f & py::array::f_style))
        throw py::value_error(std::string(name) + " must be C- or Fortran-contiguous");
}

void check_out(const py::array &a, const char *name, const py::dtype &dt, int64_t need_bytes) {
    check_contiguous(a, name);
    if (!a.dtype().is(dt)) throw py::value_error(std::string(name) + " has the wrong dtype");
    if (!a.writeable()) throw py::value_error(std::string(name) + " must be writeable");
    if (a.nbytes() < need_bytes)
        throw py::value_error(std::string(name) + " holds " + std::to_string(a.nbytes()) + " bytes, needs " +
                              std::to_string(need_bytes));
}

}  // namespace

PYBIND11_MODULE(mm_q4_0_q8_1_me, m) {
    m.doc() = "Q4_0 weight x Q8_1 activation matmul (gfx950 HIP)";
    m.def(
        "mmq",
        [](py::array_t<uint8_t> weight, py::array_t<float> input, py::array quant_buf, py::array output,
           std::vector<int> input_dims, int nrows_out, int ncols_k) {
            check_contiguous(weight, "weight_q4_0");
            check_contiguous(input, "input");
            std::vector<int64_t> d(input_dims.begin(), input_dims.end());
            if (d.empty() || d.size() > 4) throw py::value_error("input_dims must hold 1..4 entries");
            int64_t T = 1;
            for (size_t i = 1; i < d.size(); ++i) T *= d[i];
            if (ncols_k > 0 && nrows_out > 0 && ncols_k % 128 == 0 && d[0] == ncols_k) {
                const int64_t w_need = (int64_t)nrows_out * (ncols_k / 32) * 18;
                if (weight.nbytes() < w_need) throw py::value_error("weight_q4_0 is smaller than nrows_out*ncols_k/32*18 bytes");
                if (input.size() < d[0] * T) throw py::value_error("input has fewer elements than prod(input_dims)");
                check_out(quant_buf, "quant_workspace", py::dtype::of<uint8_t>(), T * (ncols_k / 128) * 144);
                check_out(output, "output", py::dtype::of<float>(), (int64_t)nrows_out * T * 4);
            }
            const void *w = weight.data();
            const float *x = input.data();
            uint8_t *q = static_cast<uint8_t *>(quant_buf.mutable_data());
            float *y = static_cast<float *>(output.mutable_data());
            int rc;
            {
                py::gil_scoped_release nogil;
                rc = mat_mul_q4_0_q8_1(w, x, q, y, d.data(), (int)d.size(), nrows_out, ncols_k);
            }
            if (rc == JJO_ERR_INVALID_ARG) throw py::value_error(std::string("mat_mul_q4_0_q8_1: ") + jjo_last_error());
            if (rc != JJO_OK) throw std::runtime_error(std::string("mat_mul_q4_0_q8_1: ") + jjo_last_error());
        },
        py::arg("weight_q4_0"), py::arg("input"), py::arg("quant_workspace"), py::arg("output"),
        py::arg("input_dims"), py::arg("nrows_out"), py::arg("ncols_k"),
        "Q4_0 weight x float activation (quantize via q8_1) -> float output");
}
