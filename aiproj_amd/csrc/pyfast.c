/*
 * Fast-call Python bindings of the per-step C-ABI entry points of libkvfp8.so.
 *
 * ctypes converts each argument through Python-level type objects, which costs
 * about 4.7 us for the 27 arguments of a decode call. These METH_FASTCALL wrappers
 * convert the same arguments in C and call the same exported functions (declared in
 * include/kvfp8.h), so an eager decode step spends that much less host time before
 * its launches. Arguments keep the order of the C functions: Python ints for
 * pointers (Tensor.data_ptr(), None for a null pointer), sizes, strides and dtype
 * codes, and a float for the softmax scale. Each wrapper returns the C return code.
 *
 * Like ctypes, each wrapper releases the GIL around the C call: a call can block (the
 * first call on a device queries device attributes and symbol addresses, and a launch
 * waits when the stream's queue is full), and other Python threads keep running then.
 *
 * Built by aiproj_amd/build.py with the host C compiler against the Python headers,
 * linked to libkvfp8.so in the same directory.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

#include "../../include/kvfp8.h"

/* args[0..n) as int64 (None -> 0), except the one at float_at (when >= 0), which
   goes to *fv as a float. */
static int parse(PyObject* const* args, Py_ssize_t nargs, Py_ssize_t n, Py_ssize_t float_at, int64_t* iv,
                 float* fv, const char* name) {
    if (nargs != n) {
        PyErr_Format(PyExc_TypeError, "%s takes %zd arguments (%zd given)", name, n, nargs);
        return 0;
    }
    for (Py_ssize_t i = 0; i < n; ++i) {
        PyObject* o = args[i];
        if (i == float_at) {
            const double d = PyFloat_AsDouble(o);
            if (d == -1.0 && PyErr_Occurred()) return 0;
            *fv = (float)d;
            iv[i] = 0;
        } else if (o == Py_None) {
            iv[i] = 0;
        } else {
            const long long v = PyLong_AsLongLong(o);
            if (v == -1 && PyErr_Occurred()) return 0;
            iv[i] = (int64_t)v;
        }
    }
    return 1;
}

#define PTR(i) ((void*)(uintptr_t)iv[i])

/* The 27 arguments shared by the decode entry points (float at index 22). */
#define DECODE_N 27
#define DECODE_ARGS                                                                                         \
    PTR(0), (int)iv[1], iv[2], iv[3], (int32_t)iv[4], (int32_t)iv[5], (int32_t)iv[6], (int32_t)iv[7],        \
        PTR(8), PTR(9), (int)iv[10], (const float*)PTR(11), (const float*)PTR(12), iv[13], (int32_t)iv[14], \
        (const int32_t*)PTR(15), iv[16], iv[17], PTR(18), (int)iv[19], PTR(20), (int)iv[21], scale, PTR(23), \
        PTR(24), iv[25], PTR(26)

#define DECODE_WRAPPER(fn)                                                                   \
    static PyObject* py_##fn(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {      \
        (void)self;                                                                          \
        int64_t iv[DECODE_N];                                                                \
        float scale = 0.0f;                                                                  \
        if (!parse(args, nargs, DECODE_N, 22, iv, &scale, #fn)) return NULL;                 \
        int rc;                                                                              \
        Py_BEGIN_ALLOW_THREADS                                                               \
        rc = fn(DECODE_ARGS);                                                                \
        Py_END_ALLOW_THREADS                                                                 \
        return PyLong_FromLong(rc);                                                          \
    }

DECODE_WRAPPER(kvfp8_paged_decode)
DECODE_WRAPPER(kvfp8_paged_decode_split)
DECODE_WRAPPER(kvfp8_paged_decode_reduce)

/* kvfp8_append_paged_decode: the decode arguments, then the 12 of the new rows. */
static PyObject* py_kvfp8_append_paged_decode(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
    (void)self;
    int64_t iv[DECODE_N + 12];
    float scale = 0.0f;
    if (!parse(args, nargs, DECODE_N + 12, 22, iv, &scale, "kvfp8_append_paged_decode")) return NULL;
    int rc;
    Py_BEGIN_ALLOW_THREADS
    rc = kvfp8_append_paged_decode(DECODE_ARGS, PTR(27), PTR(28), (int)iv[29], iv[30], iv[31], iv[32], iv[33],
                                   PTR(34), (int)iv[35], PTR(36), (int)iv[37], (int32_t*)PTR(38));
    Py_END_ALLOW_THREADS
    return PyLong_FromLong(rc);
}

/* kvfp8_quantize_append: 21 arguments. */
static PyObject* py_kvfp8_quantize_append(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
    (void)self;
    int64_t iv[21];
    if (!parse(args, nargs, 21, -1, iv, NULL, "kvfp8_quantize_append")) return NULL;
    int rc;
    Py_BEGIN_ALLOW_THREADS
    rc = kvfp8_quantize_append(PTR(0), PTR(1), (int)iv[2], iv[3], iv[4], iv[5], iv[6], PTR(7), (int)iv[8], PTR(9),
                               (int)iv[10], iv[11], (int32_t)iv[12], (int32_t)iv[13], iv[14], (int32_t)iv[15],
                               PTR(16), PTR(17), (float*)PTR(18), (float*)PTR(19), PTR(20));
    Py_END_ALLOW_THREADS
    return PyLong_FromLong(rc);
}

/* kvfp8_store_append: 20 arguments. */
static PyObject* py_kvfp8_store_append(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
    (void)self;
    int64_t iv[20];
    if (!parse(args, nargs, 20, -1, iv, NULL, "kvfp8_store_append")) return NULL;
    int rc;
    Py_BEGIN_ALLOW_THREADS
    rc = kvfp8_store_append(PTR(0), PTR(1), (int)iv[2], iv[3], iv[4], iv[5], iv[6], PTR(7), (int)iv[8], PTR(9),
                            (int)iv[10], iv[11], (int32_t)iv[12], (int32_t)iv[13], iv[14], (int32_t)iv[15], PTR(16),
                            PTR(17), (int)iv[18], PTR(19));
    Py_END_ALLOW_THREADS
    return PyLong_FromLong(rc);
}

static PyMethodDef methods[] = {
    {"kvfp8_paged_decode", (PyCFunction)(void (*)(void))py_kvfp8_paged_decode, METH_FASTCALL, NULL},
    {"kvfp8_paged_decode_split", (PyCFunction)(void (*)(void))py_kvfp8_paged_decode_split, METH_FASTCALL, NULL},
    {"kvfp8_paged_decode_reduce", (PyCFunction)(void (*)(void))py_kvfp8_paged_decode_reduce, METH_FASTCALL, NULL},
    {"kvfp8_append_paged_decode", (PyCFunction)(void (*)(void))py_kvfp8_append_paged_decode, METH_FASTCALL, NULL},
    {"kvfp8_quantize_append", (PyCFunction)(void (*)(void))py_kvfp8_quantize_append, METH_FASTCALL, NULL},
    {"kvfp8_store_append", (PyCFunction)(void (*)(void))py_kvfp8_store_append, METH_FASTCALL, NULL},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_kvfp8_fast",
                                    "Fast-call bindings of libkvfp8.so's per-step entry points.", -1, methods,
                                    NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__kvfp8_fast(void) { return PyModule_Create(&module); }
