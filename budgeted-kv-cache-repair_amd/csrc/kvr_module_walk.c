/* Module-tree walk of the packed executor's per-call qualification, as a
 * CPython extension (_kvr_walk). The executor refuses, before any device work,
 * a model whose decoder modules are in training mode, carry a per-instance
 * forward, a dispatch hook or a parameter off the request device, and takes
 * the module path when a decoder module carries forward hooks (the
 * reference's _qualify, src/kv_cache_repair/kernels/packed_cache.py:123-155,
 * makes the same checks over model.modules()). It also fingerprints the tree (module and parameter identities,
 * parameter storage addresses) so per-model plans can be reused while the tree
 * is unchanged. The walk visits every module of an 8B model (~420) and its
 * ~290 parameter slots on every refresh: one pass in C instead of several
 * Python passes.
 *
 * qualify_walk(model, base, data_ptr) -> (training, overridden, hooked,
 *     forward_hooked, params, dict_ids, param_ids, ptrs)
 *   inner = instance dicts of `base` and every module under it, level by
 *           level through the `_modules` dicts (None entries left out);
 *   outer = the same from `model`, leaving out the subtree of `base`;
 *   training       = any inner dict's "training" is true;
 *   overridden     = some inner dict holds "forward";
 *   hooked         = some dict (inner or outer) holds a non-None "_hf_hook";
 *   forward_hooked = some inner dict's "_forward_hooks" or
 *                    "_forward_pre_hooks" is nonempty;
 *   params         = the values of every dict's "_parameters" dict (inner then
 *                    outer, dict order; empty slots are None);
 *   dict_ids / param_ids = id() of each dict / each params entry;
 *   ptrs           = data_ptr(p) for every non-None parameter.
 * A missing "_modules", "training", "_forward_hooks", "_forward_pre_hooks" or
 * "_parameters" entry raises KeyError, as the dict lookups they replace do.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

static PyObject *s_dict, *s_modules, *s_parameters, *s_training, *s_forward, *s_hf_hook, *s_fwd_hooks,
    *s_fwd_pre_hooks;

static int append_dict(PyObject* out, PyObject* module) {
    PyObject* d = PyObject_GetAttr(module, s_dict);
    if (!d) return -1;
    if (!PyDict_Check(d)) {
        Py_DECREF(d);
        PyErr_SetString(PyExc_TypeError, "module __dict__ is not a dict");
        return -1;
    }
    const int rc = PyList_Append(out, d);
    Py_DECREF(d);
    return rc;
}

/* borrowed d[key]; KeyError when absent */
static PyObject* item(PyObject* d, PyObject* key) {
    PyObject* v = PyDict_GetItemWithError(d, key);
    if (!v && !PyErr_Occurred()) PyErr_SetObject(PyExc_KeyError, key);
    return v;
}

/* Appends to `out` the instance dicts of `root` and every module under it,
 * level by level (breadth first), skipping None entries and `skip`. A
 * `_modules` that is not exactly a dict is read through its values(). */
static int subtree(PyObject* root, PyObject* skip, PyObject* out) {
    Py_ssize_t i = PyList_GET_SIZE(out);
    if (append_dict(out, root)) return -1;
    for (; i < PyList_GET_SIZE(out); ++i) {
        PyObject* mods = item(PyList_GET_ITEM(out, i), s_modules);
        if (!mods) return -1;
        if (PyDict_CheckExact(mods)) {
            Py_ssize_t pos = 0;
            PyObject *key, *m;
            while (PyDict_Next(mods, &pos, &key, &m))
                if (m != Py_None && m != skip && append_dict(out, m)) return -1;
            continue;
        }
        PyObject* vals = PyMapping_Values(mods);
        if (!vals) return -1;
        for (Py_ssize_t j = 0; j < PyList_GET_SIZE(vals); ++j) {
            PyObject* m = PyList_GET_ITEM(vals, j);
            if (m != Py_None && m != skip && append_dict(out, m)) {
                Py_DECREF(vals);
                return -1;
            }
        }
        Py_DECREF(vals);
    }
    return 0;
}

static PyObject* qualify_walk(PyObject* self, PyObject* args) {
    PyObject *model, *base, *data_ptr;
    if (!PyArg_ParseTuple(args, "OOO:qualify_walk", &model, &base, &data_ptr)) return NULL;
    PyObject *dicts = PyList_New(0), *params = PyList_New(0), *dict_ids = NULL, *param_ids = NULL, *ptrs = NULL;
    PyObject* result = NULL;
    int training = 0, overridden = 0, hooked = 0, forward_hooked = 0;
    if (!dicts || !params) goto done;
    if (subtree(base, Py_None, dicts)) goto done;
    const Py_ssize_t n_inner = PyList_GET_SIZE(dicts);
    if (subtree(model, base, dicts)) goto done;
    const Py_ssize_t n = PyList_GET_SIZE(dicts);
    if (!(dict_ids = PyTuple_New(n))) goto done;
    for (Py_ssize_t i = 0; i < n; ++i) {
        PyObject* d = PyList_GET_ITEM(dicts, i);
        PyObject* id = PyLong_FromVoidPtr(d);
        if (!id) goto done;
        PyTuple_SET_ITEM(dict_ids, i, id);
        if (i < n_inner) {
            PyObject *t = item(d, s_training), *h, *ph;
            if (!t) goto done;
            const int tv = PyObject_IsTrue(t);
            const int fv = PyDict_Contains(d, s_forward);
            if (tv < 0 || fv < 0) goto done;
            if (!(h = item(d, s_fwd_hooks)) || !(ph = item(d, s_fwd_pre_hooks))) goto done;
            const int hv = PyObject_IsTrue(h), phv = PyObject_IsTrue(ph);
            if (hv < 0 || phv < 0) goto done;
            training |= tv;
            overridden |= fv;
            forward_hooked |= hv | phv;
        }
        PyObject* hook = PyDict_GetItemWithError(d, s_hf_hook);
        if (!hook && PyErr_Occurred()) goto done;
        hooked |= hook && hook != Py_None;
        PyObject* slots = item(d, s_parameters);
        if (!slots) goto done;
        if (!PyDict_Check(slots)) {
            PyErr_SetString(PyExc_TypeError, "module _parameters is not a dict");
            goto done;
        }
        Py_ssize_t pos = 0;
        PyObject *key, *p;
        while (PyDict_Next(slots, &pos, &key, &p))
            if (PyList_Append(params, p)) goto done;
    }
    const Py_ssize_t n_params = PyList_GET_SIZE(params);
    Py_ssize_t live = 0;
    for (Py_ssize_t j = 0; j < n_params; ++j) live += PyList_GET_ITEM(params, j) != Py_None;
    if (!(param_ids = PyTuple_New(n_params)) || !(ptrs = PyTuple_New(live))) goto done;
    for (Py_ssize_t j = 0, q = 0; j < n_params; ++j) {
        PyObject* p = PyList_GET_ITEM(params, j);
        PyObject* id = PyLong_FromVoidPtr(p);
        if (!id) goto done;
        PyTuple_SET_ITEM(param_ids, j, id);
        if (p == Py_None) continue;
        PyObject* ptr = PyObject_CallOneArg(data_ptr, p);
        if (!ptr) goto done;
        PyTuple_SET_ITEM(ptrs, q++, ptr);
    }
    result = Py_BuildValue("(OOOOOOOO)", training ? Py_True : Py_False, overridden ? Py_True : Py_False,
                           hooked ? Py_True : Py_False, forward_hooked ? Py_True : Py_False, params, dict_ids,
                           param_ids, ptrs);
done:
    Py_XDECREF(dicts);
    Py_XDECREF(params);
    Py_XDECREF(dict_ids);
    Py_XDECREF(param_ids);
    Py_XDECREF(ptrs);
    return result;
}

static PyMethodDef kMethods[] = {
    {"qualify_walk", qualify_walk, METH_VARARGS,
     "qualify_walk(model, base, data_ptr) -> (training, overridden, hooked, forward_hooked, params, dict_ids, "
     "param_ids, ptrs)"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_kvr_walk",
                                     "Module-tree walk of the packed executor's qualification.", -1, kMethods};

PyMODINIT_FUNC PyInit__kvr_walk(void) {
    struct {
        PyObject** slot;
        const char* text;
    } names[] = {{&s_dict, "__dict__"},
                 {&s_modules, "_modules"},
                 {&s_parameters, "_parameters"},
                 {&s_training, "training"},
                 {&s_forward, "forward"},
                 {&s_hf_hook, "_hf_hook"},
                 {&s_fwd_hooks, "_forward_hooks"},
                 {&s_fwd_pre_hooks, "_forward_pre_hooks"}};
    for (size_t i = 0; i < sizeof(names) / sizeof(names[0]); ++i)
        if (!(*names[i].slot = PyUnicode_InternFromString(names[i].text))) return NULL;
    return PyModule_Create(&kModule);
}
