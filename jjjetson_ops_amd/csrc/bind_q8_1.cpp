// Python module `q8_1_me`: the reference's binding surface
// (src/bindings/q8_1_binding.cpp:11-44) over the C ABI of this library.
//   quantize(input: float32 ndarray, output: uint8 ndarray, dims: list[int]) -> None
//   parse(raw: uint8 ndarray, n_blocks: int) -> (qs int8[n,128], scale f32[n,4], sum f32[n,4])
// Differences from the reference, all on error paths: failures raise
// RuntimeError/ValueError instead of exiting the process, and the output
// buffer must already be a writeable uint8 array large enough (the reference
// silently wrote into a temporary copy when given another dtype).
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

void raise_status(int rc, const char *what) {
    if (rc == JJO_OK) return;
    std::string msg = std::string(what) + ": " + jjo_last_error();
    if (rc == JJO_ERR_INVALID_ARG) throw py::value_error(msg);
    throw std::runtime_error(msg);
}

}  // namespace

PYBIND11_MODULE(q8_1_me, m) {
    m.doc() = "Q8_1 activation quantizer (gfx950 HIP)";
    m.def(
        "quantize",
        [](py::array_t<float> input, py::array output, std::vector<int> dims) {
            check_contiguous(input, "input");
            check_contiguous(output, "output");
            if (!output.dtype().is(py::dtype::of<uint8_t>()))
                throw py::value_error("output must be a uint8 array");
            if (!output.writeable()) throw py::value_error("output must be writeable");
            std::vector<int64_t> d(dims.begin(), dims.end());
            const int64_t need = q8_1_output_bytes(d.data(), (int)d.size());
            if (need < 0) raise_status(JJO_ERR_INVALID_ARG, "quantize");
            int64_t n_in = 1;
            for (int64_t v : d) n_in *= v;
            if (input.size() < n_in) throw py::value_error("input has fewer elements than prod(dims)");
            if (output.nbytes() < need)
                throw py::value_error("output holds " + std::to_string(output.nbytes()) + " bytes, needs " +
                                      std::to_string(need));
            const float *in = input.data();
            uint8_t *out = static_cast<uint8_t *>(output.mutable_data());
            int rc;
            {
                py::gil_scoped_release nogil;
                rc = q8_1(in, out, d.data(), (int)d.size());
            }
            raise_status(rc, "q8_1");
        },
        py::arg("input"), py::arg("output"), py::arg("dims"), "Quantize float32 to Q8_1");

    m.def(
        "parse",
        [](py::array_t<uint8_t> raw, int64_t n_blocks) {
            if (n_blocks < 0) throw py::value_error("n_blocks must be non-negative");
            if (raw.nbytes() < n_blocks * JJO_BLOCK_Q8_1_MMQ_BYTES)
                throw py::value_error("raw buffer is smaller than n_blocks * 144 bytes");
            check_contiguous(raw, "raw");
            auto qs = py::array_t<int8_t>(std::vector<py::ssize_t>{(py::ssize_t)n_blocks, 128});
            auto scale = py::array_t<float>(std::vector<py::ssize_t>{(py::ssize_t)n_blocks, 4});
            auto sum = py::array_t<float>(std::vector<py::ssize_t>{(py::ssize_t)n_blocks, 4});
            parse_q8_1_output(raw.data(), qs.mutable_data(), scale.mutable_data(), sum.mutable_data(), n_blocks);
            return py::make_tuple(qs, scale, sum);
        },
        py::arg("raw"), py::arg("n_blocks"), "Parse raw Q8_1 output");
}
