/*
 * _hostmask: the reference's set / dict token-head arguments as a dense mask.
 *
 * PackedKVCache.evict(set), PackedKVCache.apply_reuse_mask(dict) and
 * PagedKVStore.evict_tokens(set) (shadowinfer/shadowkv/packed_kv_cache.py:
 * 666-854, paged_kv_store.py:556-698) take Python sets of (token, head) pairs
 * and dicts (token, head) -> flag, and test entries with `in` / `.get`. The
 * kernels take a uint8 [S * H] mask instead; this module fills it in one pass
 * over the container with the same membership rule:
 *
 *   an item marks entry t * H + h when it is a 2-tuple equal to (t, h) with
 *   0 <= t < S and 0 <= h < H (for a dict, when its value is also truthy).
 *
 * Elements that are ints (bool included), numpy bools, objects with
 * __index__ (numpy integers) or floats with an integral value compare equal to
 * that integer, as in Python. Items that are not 2-tuples can never equal a
 * (t, h) tuple and are skipped. A dict value's truthiness is evaluated only
 * for keys that are in-range pairs, as the reference evaluates
 * reuse_mask.get(entry) only for entries of the cache. Any other element
 * type, or a value whose truthiness raises, makes the call return None, and
 * the caller then decides item by item in Python.
 *
 * token_head_mask(items, S, H, out, is_dict) -> int (entries marked, counting
 * repeats) or None. `out` is a writable buffer of at least S * H bytes; it is
 * not cleared here.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

/* numpy's bool scalar: equal to 0 or 1, but its __index__ is deprecated
 * (a DeprecationWarning, an error under -W error), so it is read by value. */
static int is_numpy_bool(PyObject* o) {
  const char* n = Py_TYPE(o)->tp_name;
  return strcmp(n, "numpy.bool") == 0 || strcmp(n, "numpy.bool_") == 0;
}

/* 1: integral value in *out; 0: never equal to an in-range integer;
 * -1: undecided (unknown type); -2: Python error set. */
static int element_index(PyObject* o, long long* out) {
  if (is_numpy_bool(o)) {
    const int b = PyObject_IsTrue(o);
    if (b < 0) return -2;
    *out = b;
    return 1;
  }
  if (PyLong_Check(o)) {
    int overflow = 0;
    long long v = PyLong_AsLongLongAndOverflow(o, &overflow);
    if (overflow) return 0;
    if (v == -1 && PyErr_Occurred()) return -2;
    *out = v;
    return 1;
  }
  if (PyFloat_Check(o)) {
    const double d = PyFloat_AS_DOUBLE(o);
    if (!(d == floor(d)) || fabs(d) > 9.0e15) return 0; /* NaN, fractional, huge */
    *out = (long long)d;
    return 1;
  }
  if (PyIndex_Check(o)) {
    PyObject* i = PyNumber_Index(o);
    if (i == NULL) return -2;
    int overflow = 0;
    long long v = PyLong_AsLongLongAndOverflow(i, &overflow);
    Py_DECREF(i);
    if (overflow) return 0;
    if (v == -1 && PyErr_Occurred()) return -2;
    *out = v;
    return 1;
  }
  return -1;
}

/* 1: item equals the in-range pair (t, h), *entry = t * H + h; 0: it equals
 * no in-range pair; -1 undecided; -2 error. Writes nothing. */
static int item_entry(PyObject* item, long long S, long long H, long long* entry) {
  if (!PyTuple_Check(item) || PyTuple_GET_SIZE(item) != 2) return 0;
  long long t = 0, h = 0;
  int rt = element_index(PyTuple_GET_ITEM(item, 0), &t);
  if (rt < 0) return rt;
  int rh = element_index(PyTuple_GET_ITEM(item, 1), &h);
  if (rh < 0) return rh;
  if (rt == 0 || rh == 0) return 0;
  if (t < 0 || t >= S || h < 0 || h >= H) return 0;
  *entry = t * H + h;
  return 1;
}

static PyObject* token_head_mask(PyObject* self, PyObject* args) {
  (void)self;
  PyObject* items;
  long long S, H;
  Py_buffer buf;
  int is_dict;
  if (!PyArg_ParseTuple(args, "OLLw*p", &items, &S, &H, &buf, &is_dict)) return NULL;
  if (S < 0 || H < 0 || buf.len < S * H) {
    PyBuffer_Release(&buf);
    PyErr_SetString(PyExc_ValueError, "token_head_mask: buffer smaller than S * H");
    return NULL;
  }
  unsigned char* out = (unsigned char*)buf.buf;
  long long marked = 0;
  int undecided = 0;
  if (is_dict) {
    if (!PyDict_Check(items)) {
      PyBuffer_Release(&buf);
      PyErr_SetString(PyExc_TypeError, "token_head_mask: is_dict needs a dict");
      return NULL;
    }
    Py_ssize_t pos = 0;
    PyObject *key, *value;
    while (PyDict_Next(items, &pos, &key, &value)) {
      long long e = 0;
      const int r = item_entry(key, S, H, &e);
      if (r == -2) {
        PyBuffer_Release(&buf);
        return NULL;
      }
      if (r == -1) {
        undecided = 1;
        break;
      }
      if (r == 0) continue;
      const int truthy = PyObject_IsTrue(value);
      if (truthy < 0) { /* decided by the Python rule, which raises the same error */
        PyErr_Clear();
        undecided = 1;
        break;
      }
      if (!truthy) continue;
      out[e] = 1;
      marked += 1;
    }
  } else {
    PyObject* it = PyObject_GetIter(items);
    if (it == NULL) {
      PyBuffer_Release(&buf);
      return NULL;
    }
    PyObject* item;
    while ((item = PyIter_Next(it)) != NULL) {
      long long e = 0;
      const int r = item_entry(item, S, H, &e);
      Py_DECREF(item);
      if (r == 1) out[e] = 1;
      if (r == -2) {
        Py_DECREF(it);
        PyBuffer_Release(&buf);
        return NULL;
      }
      if (r == -1) {
        undecided = 1;
        break;
      }
      marked += r;
    }
    Py_DECREF(it);
    if (PyErr_Occurred()) {
      PyBuffer_Release(&buf);
      return NULL;
    }
  }
  PyBuffer_Release(&buf);
  if (undecided) Py_RETURN_NONE;
  return PyLong_FromLongLong(marked);
}

static PyMethodDef methods[] = {
    {"token_head_mask", token_head_mask, METH_VARARGS,
     "token_head_mask(items, S, H, out, is_dict) -> marked count or None"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_hostmask",
                                    "set / dict token-head arguments as a dense mask", -1,
                                    methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__hostmask(void) { return PyModule_Create(&module); }
