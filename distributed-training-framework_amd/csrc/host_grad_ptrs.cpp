// _hostptrs: one host-side helper for the DDP launch path, a CPython module
// built against torch's headers.  It is bookkeeping, not compute, and not part
// of the C ABI of libmdx.so.
//
// Before every launch of a run of buckets, DDP needs the address of each
// parameter's .grad (0 for None) to see whether its kernel tables still hold.
// In Python that is `p.grad` and `.data_ptr()` per parameter, ~150 ns each
// (about 20 us for GPT-2's 148 gradients, on the path between the previous
// step's flag read and the next launch); here it is one call.
#include <Python.h>

#include <torch/csrc/autograd/python_variable.h>

namespace {

PyObject* grad_ptrs(PyObject*, PyObject* params) {
  if (!PyList_Check(params)) {
    PyErr_SetString(PyExc_TypeError, "grad_ptrs: expected a list of parameters");
    return nullptr;
  }
  const Py_ssize_t n = PyList_GET_SIZE(params);
  PyObject* out = PyList_New(n);
  if (out == nullptr) return nullptr;
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* p = PyList_GET_ITEM(params, i);
    if (!THPVariable_Check(p)) {
      Py_DECREF(out);
      PyErr_SetString(PyExc_TypeError, "grad_ptrs: every element must be a tensor");
      return nullptr;
    }
    unsigned long long addr = 0;
    try {
      // torch's own error (a gradient without storage, e.g. a sparse one) goes back to Python as a
      // RuntimeError: an exception must not leave this C function
      const at::Tensor& g = THPVariable_Unpack(p).grad();
      if (g.defined()) addr = static_cast<unsigned long long>(reinterpret_cast<uintptr_t>(g.data_ptr()));
    } catch (const std::exception& e) {
      Py_DECREF(out);
      PyErr_SetString(PyExc_RuntimeError, e.what());
      return nullptr;
    }
    PyObject* v = PyLong_FromUnsignedLongLong(addr);
    if (v == nullptr) {
      Py_DECREF(out);
      return nullptr;
    }
    PyList_SET_ITEM(out, i, v);
  }
  return out;
}

PyMethodDef kMethods[] = {
    {"grad_ptrs", grad_ptrs, METH_O, "Address of each parameter's .grad storage (0 where .grad is None)."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_hostptrs", nullptr, -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__hostptrs(void) { return PyModule_Create(&kModule); }
