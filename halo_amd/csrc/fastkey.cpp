// Layout key of a chunk list for triton_chunked_attention's per-layout fast
// path (host code, no GPU work): for every (k, v, chunk_start, causal) the
// data address, element type, sizes and strides of k and v, then the chunk
// start and the causal flag, packed as int64s into one bytes object.  Two
// chunk lists get equal keys exactly when every one of those values is equal
// (the same fields halo_amd/triton_chunked.py's Python key reads, at about a
// quarter of the cost: the attributes are read from the tensors in C++
// instead of through one Python call each).
#include <torch/extension.h>

#include <vector>

namespace py = pybind11;

namespace {

void put_tensor(std::vector<int64_t>& w, const at::Tensor& t) {
  w.push_back(reinterpret_cast<int64_t>(t.data_ptr()));
  w.push_back(static_cast<int64_t>(t.scalar_type()));
  w.push_back(t.dim());
  for (const int64_t s : t.sizes()) w.push_back(s);
  for (const int64_t s : t.strides()) w.push_back(s);
}

py::bytes chunk_layout_key(const py::sequence& chunks) {
  std::vector<int64_t> w;
  w.reserve(chunks.size() * 24);
  for (const auto item : chunks) {
    const auto c = py::reinterpret_borrow<py::sequence>(item);
    if (c.size() != 4) throw py::type_error("chunks must be (k, v, chunk_start, causal) tuples");
    put_tensor(w, c[0].cast<at::Tensor>());
    put_tensor(w, c[1].cast<at::Tensor>());
    w.push_back(c[2].cast<int64_t>());
    w.push_back(c[3].cast<bool>() ? 1 : 0);
  }
  return py::bytes(reinterpret_cast<const char*>(w.data()), w.size() * sizeof(int64_t));
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("chunk_layout_key", &chunk_layout_key, "layout key of a (k, v, chunk_start, causal) list");
}
