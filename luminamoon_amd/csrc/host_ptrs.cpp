// Host-side helper of the optimizer's cached step plans (luminamoon_amd/optimizer/luminav.py): it
// checks that a list of tensors still has the data pointers a plan recorded, in one C loop. A
// plan of 64 tensors checks its params, grads and state tensors (about 250 tensors) before every
// step; through Python's Tensor.data_ptr each costs a method call, a quarter of a small step's
// whole host time. Not part of the step itself: the optimizer falls back to the Python
// comparison when this module is not built.
#include <Python.h>

#include <cstdint>
#include <cstring>
#include <exception>

#include <torch/csrc/autograd/python_variable.h>

namespace {

// same_ptrs(tensors: list, recorded: bytes) -> bool: len(recorded) == 8 * len(tensors) and every
// tensors[i] is a tensor whose data_ptr() equals the i-th native-endian uint64 of recorded.
PyObject *same_ptrs(PyObject *, PyObject *args) {
    PyObject *tensors = nullptr, *recorded = nullptr;
    if (!PyArg_ParseTuple(args, "O!O!", &PyList_Type, &tensors, &PyBytes_Type, &recorded)) return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(tensors);
    if (PyBytes_GET_SIZE(recorded) != n * (Py_ssize_t)sizeof(uint64_t)) Py_RETURN_FALSE;
    const char *want = PyBytes_AS_STRING(recorded);
    try {
        for (Py_ssize_t i = 0; i < n; i++) {
            PyObject *o = PyList_GET_ITEM(tensors, i);
            if (!THPVariable_Check(o)) Py_RETURN_FALSE;
            const at::Tensor &t = THPVariable_Unpack(o);
            uint64_t w;
            std::memcpy(&w, want + i * sizeof(uint64_t), sizeof w);
            if ((uint64_t)(uintptr_t)t.data_ptr() != w) Py_RETURN_FALSE;
        }
    } catch (const std::exception &e) {  // a tensor without storage: data_ptr raises, as in Python
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    Py_RETURN_TRUE;
}

// ptrs(tensors: list) -> bytes: the data pointers as native-endian uint64 (what same_ptrs reads).
PyObject *ptrs(PyObject *, PyObject *args) {
    PyObject *tensors = nullptr;
    if (!PyArg_ParseTuple(args, "O!", &PyList_Type, &tensors)) return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(tensors);
    PyObject *out = PyBytes_FromStringAndSize(nullptr, n * (Py_ssize_t)sizeof(uint64_t));
    if (!out) return nullptr;
    char *dst = PyBytes_AS_STRING(out);
    try {
        for (Py_ssize_t i = 0; i < n; i++) {
            PyObject *o = PyList_GET_ITEM(tensors, i);
            if (!THPVariable_Check(o)) {
                Py_DECREF(out);
                PyErr_SetString(PyExc_TypeError, "ptrs: a list of tensors is expected");
                return nullptr;
            }
            const uint64_t p = (uint64_t)(uintptr_t)THPVariable_Unpack(o).data_ptr();
            std::memcpy(dst + i * sizeof(uint64_t), &p, sizeof p);
        }
    } catch (const std::exception &e) {
        Py_DECREF(out);
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    return out;
}

PyMethodDef kMethods[] = {
    {"same_ptrs", same_ptrs, METH_VARARGS, "Do these tensors still have the recorded data pointers?"},
    {"ptrs", ptrs, METH_VARARGS, "The tensors' data pointers as packed uint64."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_lv_host", "Data-pointer checks of the optimizer's step plans.", -1,
                       kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__lv_host(void) { return PyModule_Create(&kModule); }
