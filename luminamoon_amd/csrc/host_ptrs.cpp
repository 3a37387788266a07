// Host-side helper of the optimizer's cached step plans (luminamoon_amd/optimizer/luminav.py): it
// checks that a list of tensors still has the data pointers a plan recorded, in one C loop. A
// plan of 64 tensors checks its params, grads and state tensors (about 250 tensors) before every
// step; through Python's Tensor.data_ptr each costs a method call, a quarter of a small step's
// whole host time. `grad_record` makes all of a step's checks of a plan whose every param has a
// grad in one call and records where the grads are, and `advance` moves the step counters. Not
// part of the step itself: the optimizer falls back to Python when this module is not built.
#include <Python.h>

#include <cstdint>
#include <cstring>
#include <exception>

#include <torch/csrc/Dtype.h>
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

// Reads the i-th native-endian uint64 of a bytes record.
inline uint64_t rec(PyObject *b, Py_ssize_t i) {
    uint64_t w;
    std::memcpy(&w, PyBytes_AS_STRING(b) + i * sizeof(uint64_t), sizeof w);
    return w;
}

// advance(states: list of dict, steps: list of int, key: str) -> list: the counters plus one, each
// also stored under `key` in its state dict (dict.__setitem__, as the Python path does).
PyObject *advance(PyObject *, PyObject *args) {
    PyObject *states = nullptr, *steps = nullptr, *key = nullptr;
    if (!PyArg_ParseTuple(args, "O!O!U", &PyList_Type, &states, &PyList_Type, &steps, &key)) return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(states);
    if (PyList_GET_SIZE(steps) != n) {
        PyErr_SetString(PyExc_ValueError, "advance: as many counters as states are expected");
        return nullptr;
    }
    PyObject *out = PyList_New(n);
    if (!out) return nullptr;
    for (Py_ssize_t i = 0; i < n; i++) {
        PyObject *d = PyList_GET_ITEM(states, i);
        if (!PyDict_Check(d)) {
            Py_DECREF(out);
            PyErr_SetString(PyExc_TypeError, "advance: a list of dicts is expected");
            return nullptr;
        }
        const long long v = PyLong_AsLongLong(PyList_GET_ITEM(steps, i));
        if (v == -1 && PyErr_Occurred()) {
            Py_DECREF(out);
            return nullptr;
        }
        PyObject *nv = PyLong_FromLongLong(v + 1);
        if (!nv || PyDict_SetItem(d, key, nv) < 0) {
            Py_XDECREF(nv);
            Py_DECREF(out);
            return nullptr;
        }
        PyList_SET_ITEM(out, i, nv);  // the list takes the reference
    }
    return out;
}

// Whether tensor t fits a descriptor of dtype `dt` (a torch.dtype, checked by the caller) with
// `want` elements on GPU `device`: dense, contiguous, on that device.
inline bool fits(const at::Tensor &t, PyObject *dt, long long want, int device) {
    return t.scalar_type() == reinterpret_cast<THPDtype *>(dt)->scalar_type && t.layout() == c10::kStrided &&
           t.is_cuda() && t.get_device() == device && t.numel() == want && t.is_contiguous();
}

// grad_record(params: list, pids: bytes, pptrs: bytes, stensors: list, sptrs: bytes, dtypes: list of
// torch.dtype, numels: list of int, device: int) -> bytes or None. For a plan whose every param has
// a grad: the grads' data pointers as packed native-endian uint64 when the params are the recorded
// objects (id(params[i]) == pids[i]) at their recorded data pointers, the state tensors are at
// theirs, and every param's grad fits its descriptor (a dense, contiguous tensor of dtypes[i] with
// numels[i] elements on GPU `device`); None otherwise (a grad of None included). Every check is
// made at every call, so a new grad object is taken as it is, wherever it lives: the plan needs no
// record of the grads' identities. Records of another length give None; malformed arguments and a
// tensor without storage raise.
PyObject *grad_record(PyObject *, PyObject *args) {
    PyObject *params = nullptr, *pids = nullptr, *pptrs = nullptr, *stensors = nullptr, *sptrs = nullptr;
    PyObject *dtypes = nullptr, *numels = nullptr;
    int device = -1;
    if (!PyArg_ParseTuple(args, "O!O!O!O!O!O!O!i", &PyList_Type, &params, &PyBytes_Type, &pids, &PyBytes_Type, &pptrs,
                          &PyList_Type, &stensors, &PyBytes_Type, &sptrs, &PyList_Type, &dtypes, &PyList_Type, &numels,
                          &device))
        return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(params);
    const Py_ssize_t bytes = n * (Py_ssize_t)sizeof(uint64_t);
    if (PyList_GET_SIZE(dtypes) != n || PyList_GET_SIZE(numels) != n) {
        PyErr_SetString(PyExc_ValueError, "grad_record: as many dtypes and sizes as params are expected");
        return nullptr;
    }
    const Py_ssize_t ns = PyList_GET_SIZE(stensors);
    if (PyBytes_GET_SIZE(pids) != bytes || PyBytes_GET_SIZE(pptrs) != bytes ||
        PyBytes_GET_SIZE(sptrs) != ns * (Py_ssize_t)sizeof(uint64_t))
        Py_RETURN_NONE;
    PyObject *out = PyBytes_FromStringAndSize(nullptr, bytes);
    if (!out) return nullptr;
    char *dst = PyBytes_AS_STRING(out);
    try {
        for (Py_ssize_t i = 0; i < ns; i++) {
            PyObject *o = PyList_GET_ITEM(stensors, i);
            if (!THPVariable_Check(o) || (uint64_t)(uintptr_t)THPVariable_Unpack(o).data_ptr() != rec(sptrs, i)) {
                Py_DECREF(out);
                Py_RETURN_NONE;
            }
        }
        for (Py_ssize_t i = 0; i < n; i++) {
            PyObject *o = PyList_GET_ITEM(params, i);
            PyObject *dt = PyList_GET_ITEM(dtypes, i);
            if (!THPDtype_Check(dt)) {
                Py_DECREF(out);
                PyErr_SetString(PyExc_TypeError, "grad_record: a list of torch.dtype is expected");
                return nullptr;
            }
            const long long want = PyLong_AsLongLong(PyList_GET_ITEM(numels, i));
            if (want == -1 && PyErr_Occurred()) {
                Py_DECREF(out);
                return nullptr;
            }
            if ((uint64_t)(uintptr_t)o != rec(pids, i) || !THPVariable_Check(o)) {
                Py_DECREF(out);
                Py_RETURN_NONE;
            }
            const at::Tensor &t = THPVariable_Unpack(o);
            const at::Tensor &g = t.grad();
            if ((uint64_t)(uintptr_t)t.data_ptr() != rec(pptrs, i) || !g.defined() || !fits(g, dt, want, device)) {
                Py_DECREF(out);
                Py_RETURN_NONE;
            }
            const uint64_t gp = (uint64_t)(uintptr_t)g.data_ptr();
            std::memcpy(dst + i * sizeof(uint64_t), &gp, sizeof gp);
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
    {"advance", advance, METH_VARARGS, "The step counters plus one, also stored in the state dicts."},
    {"grad_record", grad_record, METH_VARARGS, "Checks of a plan's params, grads and state; where its grads are."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_lv_host", "Data-pointer checks of the optimizer's step plans.", -1,
                       kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__lv_host(void) { return PyModule_Create(&kModule); }
