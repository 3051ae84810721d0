// fastmoe_amd._host: host-side helpers of the Python operator layer (not part of the C ABI).
//
// The autograd combine is called with hundreds of expert buffers, and every call validates them
// and packs their (address, rows) pairs for the C ABI (prepare_grouped_metadata's Python loop over
// the tensors, src/fastmoe/kernels/ops.py:221-234, does the same job in the reference).  Read
// through Python accessors that costs about 0.25 us per tensor and property; this module reads
// the same properties from the tensors' C++ objects in one pass.  It only inspects tensors and
// writes host memory: no device memory is touched and no HIP call is made.
//
//   experts(seq, versions=False) -> (hidden, n_rows, max_rows, table, version_sum)
//       Every element must be a tensor with the dtype and device of seq[0], 2-D with seq[0]'s
//       column count, and row-contiguous (is_contiguous()).  table is a bytearray of 16 * E bytes:
//       the E data addresses (int64; 0 for an expert without rows), then the E row counts.
//       version_sum is versions(seq) when asked for, else 0.
//   versions(seq) -> int
//       Sum of the tensors' autograd version counters.  Counters never decrease, so the sum
//       grows whenever any tensor is modified in place.
#include <Python.h>

#include <cstdint>
#include <cstring>
#include <string>

#include <torch/csrc/autograd/python_variable.h>

namespace {

PyObject* raise_at(PyObject* type, Py_ssize_t i, const std::string& what) {
  const std::string msg = "fastmoe_amd: expert_tensors[" + std::to_string(i) + "] " + what;
  PyErr_SetString(type, msg.c_str());
  return nullptr;
}

std::string dims(c10::IntArrayRef v) {
  std::string s = "(";
  for (size_t i = 0; i < v.size(); ++i) {
    if (i) s += ", ";
    s += std::to_string(v[i]);
  }
  return s + (v.size() == 1 ? ",)" : ")");
}

PyObject* experts(PyObject*, PyObject* args) {
  PyObject* seq = nullptr;
  int with_versions = 0;
  if (!PyArg_ParseTuple(args, "O|p", &seq, &with_versions)) return nullptr;
  PyObject* fast = PySequence_Fast(seq, "fastmoe_amd: expert_tensors must be a sequence");
  if (!fast) return nullptr;
  const Py_ssize_t E = PySequence_Fast_GET_SIZE(fast);
  if (E == 0) {
    Py_DECREF(fast);
    PyErr_SetString(PyExc_ValueError, "fastmoe_amd: expert_tensors is empty");
    return nullptr;
  }
  PyObject* table = PyByteArray_FromStringAndSize(nullptr, 16 * E);
  if (!table) {
    Py_DECREF(fast);
    return nullptr;
  }
  int64_t* ptrs = reinterpret_cast<int64_t*>(PyByteArray_AS_STRING(table));
  int64_t* rows = ptrs + E;
  PyObject** items = PySequence_Fast_ITEMS(fast);
  PyObject* err = nullptr;
  int64_t hidden = 0, total = 0, max_rows = 0;
  long long version_sum = 0;
  at::ScalarType dtype = at::ScalarType::Undefined;
  c10::Device device(c10::DeviceType::CPU);
  try {
  for (Py_ssize_t i = 0; i < E && !err; ++i) {
    if (!THPVariable_Check(items[i])) {
      err = raise_at(PyExc_TypeError, i, "is not a tensor");
      break;
    }
    const at::Tensor& t = THPVariable_Unpack(items[i]);
    if (t.layout() != c10::kStrided) {
      err = raise_at(PyExc_ValueError, i, "must be a dense (strided) tensor");
      break;
    }
    if (i == 0) {
      dtype = t.scalar_type();
      device = t.device();
      if (t.dim() != 2) {
        err = raise_at(PyExc_ValueError, i,
                       "must be 2-D [rows, D], got shape " + dims(t.sizes()));
        break;
      }
      hidden = t.size(1);
    }
    if (t.scalar_type() != dtype || t.device() != device) {
      err = raise_at(PyExc_ValueError, i, "differs in device/dtype from [0]");
    } else if (t.dim() != 2 || t.size(1) != hidden) {
      err = raise_at(PyExc_ValueError, i,
                     "has shape " + dims(t.sizes()) + ", expected [*, " + std::to_string(hidden) +
                         "]");
    } else if (!t.is_contiguous()) {
      err = raise_at(PyExc_ValueError, i,
                     "must be row-contiguous (strides " + dims(t.strides()) + ")");
    } else {
      const int64_t n = t.size(0);
      ptrs[i] = n ? reinterpret_cast<int64_t>(t.data_ptr()) : 0;
      rows[i] = n;
      total += n;
      if (n > max_rows) max_rows = n;
      if (with_versions) version_sum += (long long)t._version();
    }
  }
  } catch (const std::exception& e) {  // a tensor type whose accessors throw
    PyErr_SetString(PyExc_ValueError, e.what());
  }
  Py_DECREF(fast);
  if (err || PyErr_Occurred()) {
    Py_DECREF(table);
    return nullptr;
  }
  // "O" takes a new reference to table on success and none on failure, so ours is dropped
  // either way.
  PyObject* res = Py_BuildValue("(LLLOL)", (long long)hidden, (long long)total,
                                (long long)max_rows, table, version_sum);
  Py_DECREF(table);
  return res;
}

PyObject* versions(PyObject*, PyObject* seq) {
  PyObject* fast = PySequence_Fast(seq, "fastmoe_amd: expected a sequence of tensors");
  if (!fast) return nullptr;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(fast);
  PyObject** items = PySequence_Fast_ITEMS(fast);
  long long sum = 0;
  try {
    for (Py_ssize_t i = 0; i < n; ++i) {
      if (!THPVariable_Check(items[i])) {
        PyErr_SetString(PyExc_TypeError, "fastmoe_amd: expected a sequence of tensors");
        break;
      }
      sum += (long long)THPVariable_Unpack(items[i])._version();
    }
  } catch (const std::exception& e) {  // e.g. an inference tensor, which has no version counter
    PyErr_SetString(PyExc_ValueError, e.what());
  }
  Py_DECREF(fast);
  if (PyErr_Occurred()) return nullptr;
  return PyLong_FromLongLong(sum);
}

PyMethodDef kMethods[] = {
    {"experts", experts, METH_VARARGS,
     "experts(seq, versions=False) -> (hidden, n_rows, max_rows, table, version_sum): validate "
     "the expert buffers and pack their (address, rows) pairs"},
    {"versions", versions, METH_O, "versions(seq) -> sum of the tensors' version counters"},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_host",
                       "Host-side helpers of fastmoe_amd's operator layer", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__host(void) { return PyModule_Create(&kModule); }
