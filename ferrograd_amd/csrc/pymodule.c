/* _fgc: the hot methods of the Python Tensor (ferrograd_amd.Tensor) as a
 * CPython extension type over the C-ABI in include/ferrograd.h.
 *
 * Building a lazy graph from Python calls one C-ABI function per op
 * (tensor.rs:442-778); through ctypes each call costs about 1.5-2 us of
 * argument conversion and wrapper objects on top of the op itself, which
 * made a Python-driven realise of ((x*0.5)+1).relu().sum(1) host-bound. Here
 * each op is one C call from the interpreter: the handle lives in the object,
 * results are new objects of the caller's type, and errors raise the
 * package's FerrogradError with fg_last_error()'s message. Everything else
 * (construction from host data, reads, autograd entry points) stays in the
 * Python class, which subclasses this type. */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include "ferrograd.h"

static PyObject* g_error_class = NULL; /* FerrogradError, registered by the package */

typedef struct {
  PyObject_HEAD fg_tensor* h;
  PyObject* weakrefs;
} TensorObject;

static PyObject* raise_last(void) {
  PyErr_SetString(g_error_class ? g_error_class : PyExc_RuntimeError, fg_last_error());
  return NULL;
}

/* A new object of `tp` owning handle `h`. */
static PyObject* wrap(PyTypeObject* tp, fg_tensor* h) {
  TensorObject* o = (TensorObject*)tp->tp_alloc(tp, 0);
  if (!o) {
    fg_tensor_free(h);
    return NULL;
  }
  o->h = h;
  return (PyObject*)o;
}

static int check_tensor(PyObject* o, TensorObject** out);

/* Every op needs a handle: Tensor() without one is an empty shell. */
static int has_handle(TensorObject* t) {
  if (t->h) return 1;
  PyErr_SetString(g_error_class ? g_error_class : PyExc_RuntimeError, "tensor has no handle");
  return 0;
}

static void t_dealloc(TensorObject* self) {
  if (self->weakrefs) PyObject_ClearWeakRefs((PyObject*)self);
  if (self->h) fg_tensor_free(self->h);
  self->h = NULL;
  Py_TYPE(self)->tp_free((PyObject*)self);
}

/* Tensor(handle): adopt a handle the C-ABI returned (an int or None). */
static int t_init(TensorObject* self, PyObject* args, PyObject* kw) {
  PyObject* hv = Py_None;
  if (!PyArg_ParseTuple(args, "|O", &hv)) return -1;
  if (self->h) {
    fg_tensor_free(self->h);
    self->h = NULL;
  }
  if (hv == Py_None) return 0;
  void* p = PyLong_AsVoidPtr(hv);
  if (!p && PyErr_Occurred()) return -1;
  self->h = (fg_tensor*)p;
  return 0;
}

static PyObject* t_get_h(TensorObject* self, void* closure) {
  (void)closure;
  if (!self->h) Py_RETURN_NONE;
  return PyLong_FromVoidPtr(self->h);
}

static PyObject* unary(TensorObject* self, int op) {
  if (!has_handle(self)) return NULL;
  fg_tensor* out = NULL;
  if (fg_tensor_unary(self->h, op, &out)) return raise_last();
  return wrap(Py_TYPE(self), out);
}

static PyObject* binary(TensorObject* self, PyObject* other, int op) {
  TensorObject* o;
  if (check_tensor(other, &o) || !has_handle(self) || !has_handle(o)) return NULL;
  fg_tensor* out = NULL;
  if (fg_tensor_binary(self->h, o->h, op, &out)) return raise_last();
  return wrap(Py_TYPE(self), out);
}

/* A sequence of ints as int64 (at most 16: tensors here have few dims). */
static int int64s(PyObject* seq, int64_t* buf, int* n) {
  PyObject* f = PySequence_Fast(seq, "expected a sequence of ints");
  if (!f) return -1;
  Py_ssize_t len = PySequence_Fast_GET_SIZE(f);
  if (len > 16) {
    Py_DECREF(f);
    PyErr_SetString(PyExc_ValueError, "at most 16 dimensions");
    return -1;
  }
  for (Py_ssize_t i = 0; i < len; i++) {
    long long v = PyLong_AsLongLong(PySequence_Fast_GET_ITEM(f, i));
    if (v == -1 && PyErr_Occurred()) {
      Py_DECREF(f);
      return -1;
    }
    buf[i] = (int64_t)v;
  }
  *n = (int)len;
  Py_DECREF(f);
  return 0;
}

static PyObject* reduce(TensorObject* self, PyObject* axes, int op) {
  if (!has_handle(self)) return NULL;
  int64_t a[16];
  int n = 0;
  if (int64s(axes, a, &n)) return NULL;
  fg_tensor* out = NULL;
  if (fg_tensor_reduce(self->h, op, a, n, &out)) return raise_last();
  return wrap(Py_TYPE(self), out);
}

static PyObject* movement(TensorObject* self, PyObject* arg, int op) {
  if (!has_handle(self)) return NULL;
  int64_t a[16];
  int n = 0;
  if (int64s(arg, a, &n)) return NULL;
  fg_tensor* out = NULL;
  if (fg_tensor_movement(self->h, op, a, n, &out)) return raise_last();
  return wrap(Py_TYPE(self), out);
}

#define UNARY(name, op) \
  static PyObject* t_##name(TensorObject* self, PyObject* unused) { (void)unused; return unary(self, op); }
UNARY(neg, FG_UNARY_NEG)
UNARY(reciprocal, FG_UNARY_RECIPROCAL)
UNARY(exp2, FG_UNARY_EXP2)
UNARY(log2, FG_UNARY_LOG2)
UNARY(sqrt, FG_UNARY_SQRT)
UNARY(relu, FG_UNARY_RELU)
UNARY(exp, FG_UNARY_EXP)
UNARY(log, FG_UNARY_LOG)
UNARY(contiguous, FG_UNARY_CONTIGUOUS)
UNARY(detach, FG_UNARY_DETACH)
UNARY(alias, FG_UNARY_ALIAS)

#define BINARY(name, op) \
  static PyObject* t_##name(TensorObject* self, PyObject* other) { return binary(self, other, op); }
BINARY(add, FG_BINARY_ADD)
BINARY(mul, FG_BINARY_MUL)
BINARY(sub, FG_BINARY_SUB)
BINARY(matmul, FG_BINARY_MATMUL)
BINARY(cross_entropy, FG_BINARY_CROSS_ENTROPY)

static PyObject* t_sum(TensorObject* self, PyObject* axes) { return reduce(self, axes, FG_REDUCE_SUM); }
static PyObject* t_max(TensorObject* self, PyObject* axes) { return reduce(self, axes, FG_REDUCE_MAX); }
static PyObject* t_reshape(TensorObject* self, PyObject* s) { return movement(self, s, FG_MOVE_RESHAPE); }
static PyObject* t_permute(TensorObject* self, PyObject* s) { return movement(self, s, FG_MOVE_PERMUTE); }
static PyObject* t_expand(TensorObject* self, PyObject* s) { return movement(self, s, FG_MOVE_EXPAND); }

static PyObject* t_u(TensorObject* self, PyObject* op) {
  long v = PyLong_AsLong(op);
  if (v == -1 && PyErr_Occurred()) return NULL;
  return unary(self, (int)v);
}

static PyObject* t_b(TensorObject* self, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 2) {
    PyErr_SetString(PyExc_TypeError, "_b(other, op)");
    return NULL;
  }
  long v = PyLong_AsLong(args[1]);
  if (v == -1 && PyErr_Occurred()) return NULL;
  return binary(self, args[0], (int)v);
}

static PyObject* t_narrow(TensorObject* self, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 3) {
    PyErr_SetString(PyExc_TypeError, "narrow(dim, start, length)");
    return NULL;
  }
  if (!has_handle(self)) return NULL;
  long long v[3];
  for (int i = 0; i < 3; i++) {
    v[i] = PyLong_AsLongLong(args[i]);
    if (v[i] == -1 && PyErr_Occurred()) return NULL;
  }
  fg_tensor* out = NULL;
  if (fg_tensor_narrow(self->h, v[0], v[1], v[2], &out)) return raise_last();
  return wrap(Py_TYPE(self), out);
}

static PyObject* t_log_softmax(TensorObject* self, PyObject* axis) {
  if (!has_handle(self)) return NULL;
  long long a = PyLong_AsLongLong(axis);
  if (a == -1 && PyErr_Occurred()) return NULL;
  fg_tensor* out = NULL;
  if (fg_tensor_log_softmax(self->h, a, &out)) return raise_last();
  return wrap(Py_TYPE(self), out);
}

static PyObject* t_realize(TensorObject* self, PyObject* unused) {
  (void)unused;
  if (!has_handle(self)) return NULL;
  if (fg_tensor_realize_many(&self->h, 1)) return raise_last();
  Py_INCREF(self);
  return (PyObject*)self;
}

static PyObject* t_assign(TensorObject* self, PyObject* other) {
  TensorObject* o;
  if (check_tensor(other, &o) || !has_handle(self) || !has_handle(o)) return NULL;
  if (fg_tensor_assign(self->h, o->h)) return raise_last();
  Py_INCREF(self);
  return (PyObject*)self;
}

static PyMethodDef t_methods[] = {
    {"neg", (PyCFunction)t_neg, METH_NOARGS, NULL},
    {"reciprocal", (PyCFunction)t_reciprocal, METH_NOARGS, NULL},
    {"exp2", (PyCFunction)t_exp2, METH_NOARGS, NULL},
    {"log2", (PyCFunction)t_log2, METH_NOARGS, NULL},
    {"sqrt", (PyCFunction)t_sqrt, METH_NOARGS, NULL},
    {"relu", (PyCFunction)t_relu, METH_NOARGS, NULL},
    {"exp", (PyCFunction)t_exp, METH_NOARGS, NULL},
    {"log", (PyCFunction)t_log, METH_NOARGS, NULL},
    {"contiguous", (PyCFunction)t_contiguous, METH_NOARGS, NULL},
    {"detach", (PyCFunction)t_detach, METH_NOARGS, NULL},
    {"alias", (PyCFunction)t_alias, METH_NOARGS, "A second handle to the same tensor identity (a Rust `clone`)."},
    {"add", (PyCFunction)t_add, METH_O, NULL},
    {"mul", (PyCFunction)t_mul, METH_O, NULL},
    {"sub", (PyCFunction)t_sub, METH_O, NULL},
    {"matmul", (PyCFunction)t_matmul, METH_O, NULL},
    {"cross_entropy", (PyCFunction)t_cross_entropy, METH_O, NULL},
    {"sum", (PyCFunction)t_sum, METH_O, NULL},
    {"max", (PyCFunction)t_max, METH_O, NULL},
    {"reshape", (PyCFunction)t_reshape, METH_O, NULL},
    {"permute", (PyCFunction)t_permute, METH_O, NULL},
    {"expand", (PyCFunction)t_expand, METH_O, NULL},
    {"narrow", (PyCFunction)(void (*)(void))t_narrow, METH_FASTCALL, NULL},
    {"log_softmax", (PyCFunction)t_log_softmax, METH_O, NULL},
    {"_u", (PyCFunction)t_u, METH_O, NULL},
    {"_b", (PyCFunction)(void (*)(void))t_b, METH_FASTCALL, NULL},
    {"realize", (PyCFunction)t_realize, METH_NOARGS, "Tensor::realize (tensor.rs:781-830)."},
    {"assign", (PyCFunction)t_assign, METH_O, "Tensor::assign (tensor.rs:421-440)."},
    {NULL, NULL, 0, NULL},
};

static PyGetSetDef t_getset[] = {
    {"_h", (getter)t_get_h, NULL, "the fg_tensor handle, as an int (None when empty)", NULL},
    {NULL, NULL, NULL, NULL, NULL},
};

static PyTypeObject TensorBaseType = {
    PyVarObject_HEAD_INIT(NULL, 0).tp_name = "ferrograd_amd._fgc.TensorBase",
    .tp_basicsize = sizeof(TensorObject),
    .tp_dealloc = (destructor)t_dealloc,
    .tp_flags = Py_TPFLAGS_DEFAULT | Py_TPFLAGS_BASETYPE,
    .tp_doc = "A lazily evaluated tensor handle (tensor.rs:95-97); the hot ops in C.",
    .tp_weaklistoffset = offsetof(TensorObject, weakrefs),
    .tp_methods = t_methods,
    .tp_getset = t_getset,
    .tp_init = (initproc)t_init,
    .tp_new = PyType_GenericNew,
};

static int check_tensor(PyObject* o, TensorObject** out) {
  if (!PyObject_TypeCheck(o, &TensorBaseType)) {
    PyErr_SetString(PyExc_TypeError, "expected a Tensor");
    return -1;
  }
  *out = (TensorObject*)o;
  return 0;
}

/* from_handle(cls, h): a `cls` owning handle h (an int). */
static PyObject* m_from_handle(PyObject* mod, PyObject* const* args, Py_ssize_t nargs) {
  (void)mod;
  if (nargs != 2 || !PyType_Check(args[0]) || !PyType_IsSubtype((PyTypeObject*)args[0], &TensorBaseType)) {
    PyErr_SetString(PyExc_TypeError, "from_handle(Tensor subclass, handle)");
    return NULL;
  }
  void* p = PyLong_AsVoidPtr(args[1]);
  if (!p) {
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_ValueError, "null tensor handle");
    return NULL;
  }
  return wrap((PyTypeObject*)args[0], (fg_tensor*)p);
}

static PyObject* m_set_error_class(PyObject* mod, PyObject* cls) {
  (void)mod;
  Py_XINCREF(cls);
  Py_XSETREF(g_error_class, cls);
  Py_RETURN_NONE;
}

static PyMethodDef m_methods[] = {
    {"from_handle", (PyCFunction)(void (*)(void))m_from_handle, METH_FASTCALL, NULL},
    {"set_error_class", (PyCFunction)m_set_error_class, METH_O, NULL},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef fgc_module = {PyModuleDef_HEAD_INIT, "_fgc", NULL, -1, m_methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__fgc(void) {
  if (PyType_Ready(&TensorBaseType) < 0) return NULL;
  PyObject* m = PyModule_Create(&fgc_module);
  if (!m) return NULL;
  Py_INCREF(&TensorBaseType);
  if (PyModule_AddObject(m, "TensorBase", (PyObject*)&TensorBaseType) < 0) {
    Py_DECREF(&TensorBaseType);
    Py_DECREF(m);
    return NULL;
  }
  return m;
}
