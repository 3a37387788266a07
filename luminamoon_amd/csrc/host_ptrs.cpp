// Host-side helper of the optimizer's cached step plans (luminamoon_amd/optimizer/luminav.py): it
// checks that a list of tensors still has the data pointers a plan recorded, in one C loop. A
// plan of 64 tensors checks its params, grads and state tensors (about 250 tensors) before every
// step; through Python's Tensor.data_ptr each costs a method call, a quarter of a small step's
// whole host time. `steady` makes all of a steady step's checks in one call (the params, their
// grads and the state tensors), `advance` moves the step counters, and `fit` checks a whole new
// set of grads and records them (after zero_grad(set_to_none=True) every step has one). Not part
// of the step itself: the optimizer falls back to Python when this module is not built.
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

// steady(params: list, pids: bytes, pptrs: bytes, gids: bytes, gptrs: bytes, stensors: list,
// sptrs: bytes) -> bool. True when the params are the recorded objects (id(params[i]) == pids[i])
// at their recorded data pointers, each has a grad that is the recorded object (id(p.grad) ==
// gids[i]) at its recorded data pointer, and the state tensors are at theirs: what a cached plan
// of a group whose every param has a grad checks before a step. False at the first difference
// (including a grad of None and a record of another length); an exception as in Python when a
// tensor has no storage.
PyObject *steady(PyObject *, PyObject *args) {
    PyObject *params = nullptr, *pids = nullptr, *pptrs = nullptr, *gids = nullptr, *gptrs = nullptr;
    PyObject *stensors = nullptr, *sptrs = nullptr;
    if (!PyArg_ParseTuple(args, "O!O!O!O!O!O!O!", &PyList_Type, &params, &PyBytes_Type, &pids, &PyBytes_Type, &pptrs,
                          &PyBytes_Type, &gids, &PyBytes_Type, &gptrs, &PyList_Type, &stensors, &PyBytes_Type, &sptrs))
        return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(params);
    const Py_ssize_t bytes = n * (Py_ssize_t)sizeof(uint64_t);
    if (PyBytes_GET_SIZE(pids) != bytes || PyBytes_GET_SIZE(pptrs) != bytes || PyBytes_GET_SIZE(gids) != bytes ||
        PyBytes_GET_SIZE(gptrs) != bytes)
        Py_RETURN_FALSE;
    const Py_ssize_t ns = PyList_GET_SIZE(stensors);
    if (PyBytes_GET_SIZE(sptrs) != ns * (Py_ssize_t)sizeof(uint64_t)) Py_RETURN_FALSE;
    try {
        for (Py_ssize_t i = 0; i < n; i++) {
            PyObject *o = PyList_GET_ITEM(params, i);
            if ((uint64_t)(uintptr_t)o != rec(pids, i) || !THPVariable_Check(o)) Py_RETURN_FALSE;
            const at::Tensor &t = THPVariable_Unpack(o);
            if ((uint64_t)(uintptr_t)t.data_ptr() != rec(pptrs, i)) Py_RETURN_FALSE;
            const at::Tensor &g = t.grad();
            if (!g.defined()) Py_RETURN_FALSE;
            PyObject *go = THPVariable_Wrap(g);  // the grad's Python object, as Tensor.grad returns it
            if (!go) return nullptr;
            const uint64_t gid = (uint64_t)(uintptr_t)go;
            Py_DECREF(go);
            if (gid != rec(gids, i) || (uint64_t)(uintptr_t)g.data_ptr() != rec(gptrs, i)) Py_RETURN_FALSE;
        }
        for (Py_ssize_t i = 0; i < ns; i++) {
            PyObject *o = PyList_GET_ITEM(stensors, i);
            if (!THPVariable_Check(o)) Py_RETURN_FALSE;
            if ((uint64_t)(uintptr_t)THPVariable_Unpack(o).data_ptr() != rec(sptrs, i)) Py_RETURN_FALSE;
        }
    } catch (const std::exception &e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    Py_RETURN_TRUE;
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

// fit(grads: list, dtypes: list of torch.dtype, numels: list of int, device: int, callback) ->
// (bytes, bytes, list) or None. None unless every grads[i] is a dense, contiguous tensor of
// dtypes[i] with numels[i] elements on GPU `device` (what a step's descriptor i accepts); else the
// grads' data pointers and their ids, each as packed native-endian uint64, and a weak reference to
// each grad with `callback`.
PyObject *fit(PyObject *, PyObject *args) {
    PyObject *grads = nullptr, *dtypes = nullptr, *numels = nullptr, *callback = nullptr;
    int device = -1;
    if (!PyArg_ParseTuple(args, "O!O!O!iO", &PyList_Type, &grads, &PyList_Type, &dtypes, &PyList_Type, &numels, &device,
                          &callback))
        return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(grads);
    if (PyList_GET_SIZE(dtypes) != n || PyList_GET_SIZE(numels) != n) {
        PyErr_SetString(PyExc_ValueError, "fit: as many dtypes and sizes as grads are expected");
        return nullptr;
    }
    PyObject *out = PyBytes_FromStringAndSize(nullptr, n * (Py_ssize_t)sizeof(uint64_t));
    if (!out) return nullptr;
    char *dst = PyBytes_AS_STRING(out);
    try {
        for (Py_ssize_t i = 0; i < n; i++) {
            PyObject *o = PyList_GET_ITEM(grads, i);
            PyObject *dt = PyList_GET_ITEM(dtypes, i);
            if (!THPDtype_Check(dt)) {
                Py_DECREF(out);
                PyErr_SetString(PyExc_TypeError, "fit: a list of torch.dtype is expected");
                return nullptr;
            }
            const long long want = PyLong_AsLongLong(PyList_GET_ITEM(numels, i));
            if (want == -1 && PyErr_Occurred()) {
                Py_DECREF(out);
                return nullptr;
            }
            if (!THPVariable_Check(o)) {  // a grad of None
                Py_DECREF(out);
                Py_RETURN_NONE;
            }
            const at::Tensor &t = THPVariable_Unpack(o);
            if (t.scalar_type() != reinterpret_cast<THPDtype *>(dt)->scalar_type || t.layout() != c10::kStrided ||
                !t.is_cuda() || t.get_device() != device || t.numel() != want || !t.is_contiguous()) {
                Py_DECREF(out);
                Py_RETURN_NONE;
            }
            const uint64_t p = (uint64_t)(uintptr_t)t.data_ptr();
            std::memcpy(dst + i * sizeof(uint64_t), &p, sizeof p);
        }
    } catch (const std::exception &e) {
        Py_DECREF(out);
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    PyObject *ids = PyBytes_FromStringAndSize(nullptr, n * (Py_ssize_t)sizeof(uint64_t));
    PyObject *refs = ids ? PyList_New(n) : nullptr;
    if (!refs) {
        Py_XDECREF(ids);
        Py_DECREF(out);
        return nullptr;
    }
    char *idst = PyBytes_AS_STRING(ids);
    for (Py_ssize_t i = 0; i < n; i++) {
        PyObject *g = PyList_GET_ITEM(grads, i);
        const uint64_t id = (uint64_t)(uintptr_t)g;
        std::memcpy(idst + i * sizeof(uint64_t), &id, sizeof id);
        PyObject *r = PyWeakref_NewRef(g, callback);
        if (!r) {
            Py_DECREF(refs);
            Py_DECREF(ids);
            Py_DECREF(out);
            return nullptr;
        }
        PyList_SET_ITEM(refs, i, r);
    }
    return Py_BuildValue("(NNN)", out, ids, refs);
}

PyMethodDef kMethods[] = {
    {"same_ptrs", same_ptrs, METH_VARARGS, "Do these tensors still have the recorded data pointers?"},
    {"ptrs", ptrs, METH_VARARGS, "The tensors' data pointers as packed uint64."},
    {"steady", steady, METH_VARARGS, "Are the params, their grads and the state tensors the recorded ones?"},
    {"advance", advance, METH_VARARGS, "The step counters plus one, also stored in the state dicts."},
    {"fit", fit, METH_VARARGS, "Check a new set of grads against the descriptors; their pointers and weak references."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_lv_host", "Data-pointer checks of the optimizer's step plans.", -1,
                       kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__lv_host(void) { return PyModule_Create(&kModule); }
