// Layout and addresses of a cache's per-layer K/V tensors in one host pass, as a
// CPython extension (_kvr_layout) reading torch's tensor metadata directly.
//
// Before the shift-cache build's launch (the reference's build_halo_cache,
// src/kv_cache_repair/cache.py:103-144, whose kernel side is
// kvr_shift_cache_build) the old cache's every layer is checked for one shared
// layout and its K and V addresses are gathered for the launch: 64 tensors at
// an 8B shape. Through Python that is ~5 attribute reads or method calls per
// tensor at ~100 ns each (~50 us in all, while the GPU waits for the launch);
// here it is one call.
//
// kv_layers(layers) -> (k_ptrs, v_ptrs, first_key, uniform)
//   for each entry of the sequence `layers`: entry.keys and entry.values (a
//   missing attribute raises AttributeError, as the attribute reads do);
//   first_key = layers[0].keys (None when there are no layers);
//   uniform   = there is at least one layer and every keys/values is a tensor
//               with first_key's sizes, strides, dtype and device and a data
//               pointer;
//   k_ptrs / v_ptrs = native uint64 data pointers of each entry's keys /
//               values (both empty when uniform is false).
// The caller applies its own checks to first_key and takes its per-tensor
// path whenever uniform is false.
//
// data_ptr(tensor) -> int
//   the tensor's data address, as torch.Tensor.data_ptr gives it, as a builtin
//   the executor's module walk calls for each of a model's ~290 parameters
//   (through Python's method descriptor each call costs several times more).
#include <Python.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>
#include <vector>

namespace {

PyObject* s_keys = nullptr;
PyObject* s_values = nullptr;

struct Layout {
    std::vector<int64_t> sizes, strides;
    caffe2::TypeMeta dtype;
    c10::Device device{c10::kCPU};
};

// true, with its data pointer in `address`, when `obj` is a tensor with
// storage and the layout `ref` (when `fill`, ref is taken from it); never throws
bool address_if_same(PyObject* obj, Layout& ref, bool fill, uint64_t& address) {
    if (!THPVariable_Check(obj)) return false;
    try {
        const at::Tensor& t = THPVariable_Unpack(obj);
        if (!t.defined() || !t.has_storage()) return false;
        if (fill) {
            ref.sizes.assign(t.sizes().begin(), t.sizes().end());
            ref.strides.assign(t.strides().begin(), t.strides().end());
            ref.dtype = t.dtype();
            ref.device = t.device();
        } else if (t.dtype() != ref.dtype || t.device() != ref.device || t.sizes() != c10::IntArrayRef(ref.sizes) ||
                   t.strides() != c10::IntArrayRef(ref.strides)) {
            return false;
        }
        address = reinterpret_cast<uint64_t>(t.const_data_ptr());
        return true;
    } catch (...) {
        return false;
    }
}

PyObject* kv_layers(PyObject*, PyObject* layers) {
    PyObject* seq = PySequence_Fast(layers, "kv_layers: layers must be a sequence");
    if (!seq) return nullptr;
    const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq);
    std::vector<uint64_t> k_ptrs(static_cast<size_t>(n)), v_ptrs(static_cast<size_t>(n));
    PyObject* first = nullptr;
    bool uniform = n > 0;
    Layout ref;
    for (Py_ssize_t i = 0; i < n; ++i) {
        PyObject* entry = PySequence_Fast_GET_ITEM(seq, i);
        PyObject* key = PyObject_GetAttr(entry, s_keys);
        if (!key) {
            Py_XDECREF(first);
            Py_DECREF(seq);
            return nullptr;
        }
        PyObject* value = PyObject_GetAttr(entry, s_values);
        if (!value) {
            Py_DECREF(key);
            Py_XDECREF(first);
            Py_DECREF(seq);
            return nullptr;
        }
        if (i == 0) {
            first = key;
            Py_INCREF(first);
        }
        if (uniform)
            uniform = address_if_same(key, ref, i == 0, k_ptrs[static_cast<size_t>(i)]) &&
                      address_if_same(value, ref, false, v_ptrs[static_cast<size_t>(i)]);
        Py_DECREF(key);
        Py_DECREF(value);
    }
    Py_DECREF(seq);
    const Py_ssize_t bytes = uniform ? 8 * n : 0;
    PyObject* kb = PyBytes_FromStringAndSize(reinterpret_cast<const char*>(k_ptrs.data()), bytes);
    PyObject* vb = PyBytes_FromStringAndSize(reinterpret_cast<const char*>(v_ptrs.data()), bytes);
    PyObject* result = nullptr;
    if (kb && vb)
        result = Py_BuildValue("(OOOO)", kb, vb, first ? first : Py_None, uniform ? Py_True : Py_False);
    Py_XDECREF(kb);
    Py_XDECREF(vb);
    Py_XDECREF(first);
    return result;
}

PyObject* data_ptr(PyObject*, PyObject* obj) {
    if (!THPVariable_Check(obj)) {
        PyErr_SetString(PyExc_TypeError, "data_ptr: expected a tensor");
        return nullptr;
    }
    try {
        // the read-only address: never materialises a copy-on-write storage
        return PyLong_FromVoidPtr(const_cast<void*>(THPVariable_Unpack(obj).const_data_ptr()));
    } catch (const std::exception& error) {
        PyErr_SetString(PyExc_RuntimeError, error.what());
        return nullptr;
    }
}

PyMethodDef kMethods[] = {
    {"kv_layers", kv_layers, METH_O, "kv_layers(layers) -> (k_ptrs, v_ptrs, first_key, uniform)"},
    {"data_ptr", data_ptr, METH_O, "data_ptr(tensor) -> int: the tensor's data address"},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_kvr_layout",
                       "Layout and addresses of a cache's per-layer K/V tensors in one pass.", -1, kMethods,
                       nullptr, nullptr, nullptr, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit__kvr_layout(void) {
    if (!(s_keys = PyUnicode_InternFromString("keys")) || !(s_values = PyUnicode_InternFromString("values")))
        return nullptr;
    return PyModule_Create(&kModule);
}
