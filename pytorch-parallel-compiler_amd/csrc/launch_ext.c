/* CPython extension _wc_launch: calls a C-ABI entry point of libwide_hip.so of the form
 *   int32_t entry(const args*, void* stream)
 * by address.  A ctypes call costs about 3 us on the host, most of a small wide forward's
 * dispatch time; this call costs a fraction of that.  The caller passes the entry point's
 * address, the address of its filled argument block and the stream handle as integers. */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

typedef int32_t (*wc_entry2)(const void*, void*);

static PyObject* call2(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (nargs != 3) {
    PyErr_SetString(PyExc_TypeError, "call2(entry, args, stream) takes 3 integer arguments");
    return NULL;
  }
  void* fn = PyLong_AsVoidPtr(args[0]);
  void* a = PyLong_AsVoidPtr(args[1]);
  void* s = PyLong_AsVoidPtr(args[2]);
  if (PyErr_Occurred()) return NULL;
  if (!fn || !a) {
    PyErr_SetString(PyExc_ValueError, "call2: null entry point or argument block");
    return NULL;
  }
  return PyLong_FromLong((long)((wc_entry2)fn)(a, s));
}

static PyMethodDef methods[] = {
    {"call2", (PyCFunction)(void (*)(void))call2, METH_FASTCALL,
     "call2(entry, args, stream) -> status: entry(args, stream) for addresses given as integers"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_wc_launch", NULL, -1, methods,
                                    NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__wc_launch(void) { return PyModule_Create(&module); }
