/*
 * _mvlaunch: CPython fast-call wrappers of the C-ABI entry points that the
 * Python wrappers call once per layer or step (mv_paged_decode_write,
 * mv_paged_decode, mv_kv_cache_write, mv_rope_kv_cache_write,
 * mv_decode_plan; include/mvattn.h).
 *
 * ctypes converts every argument through libffi: about 5 us for the 35
 * arguments of mv_paged_decode_write on the build host, a third of an eager
 * layer call's host time. These wrappers take the same arguments, in the
 * same order, as Python ints / floats / None (None: a null pointer),
 * convert them with the CPython API (under 1 us) and call the same
 * functions, through the addresses that ctypes resolved in the one loaded
 * libmvattn.so (bind()). They return the entry point's status code; the
 * caller reads mv_last_error() as for the ctypes call.
 *
 * decode_write_step takes the arguments of mv_paged_decode_write that
 * stay the same for every layer of a decode step (plan, slots, rotary
 * rows, sizes, workspace) packed once per step in a bytes object of
 * STEP_WORDS 64-bit words (step_words() below gives the order), and per
 * call only the layer's tensors: 16 arguments instead of 35.
 *
 * Host code only (plain C, no HIP): built by build_lib.build_launcher().
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include "mvattn.h"

/* The entry points' types come from the header itself: a change there that
 * this file does not follow fails the build instead of passing misordered
 * arguments. */
typedef __typeof__(&mv_paged_decode_write) decode_write_fn;
typedef __typeof__(&mv_paged_decode) decode_fn;
typedef __typeof__(&mv_kv_cache_write) cache_write_fn;
typedef __typeof__(&mv_rope_kv_cache_write) rope_write_fn;
typedef __typeof__(&mv_decode_plan) plan_fn;

static decode_write_fn g_decode_write;
static rope_write_fn g_rope_write;
static plan_fn g_plan;
static decode_fn g_decode;
static cache_write_fn g_cache_write;

/* A pointer argument: an int address, or None for a null pointer. */
static void* arg_ptr(PyObject* o) { return o == Py_None ? NULL : PyLong_AsVoidPtr(o); }
static int64_t arg_i64(PyObject* o) { return (int64_t)PyLong_AsLongLong(o); }
static int32_t arg_i32(PyObject* o) {
  const long long v = PyLong_AsLongLong(o);
  if (!PyErr_Occurred() && (v < INT32_MIN || v > INT32_MAX))
    PyErr_SetString(PyExc_OverflowError, "argument does not fit int32");
  return (int32_t)v;
}
static size_t arg_size(PyObject* o) { return (size_t)PyLong_AsUnsignedLongLong(o); }
static float arg_f32(PyObject* o) { return (float)PyFloat_AsDouble(o); }

static int check_nargs(const char* name, Py_ssize_t got, Py_ssize_t want, const void* fn) {
  if (!fn) {
    PyErr_Format(PyExc_RuntimeError, "_mvlaunch.%s: bind() was not called", name);
    return -1;
  }
  if (got != want) {
    PyErr_Format(PyExc_TypeError, "_mvlaunch.%s takes %zd arguments (%zd given)", name, want, got);
    return -1;
  }
  return 0;
}

/* Arguments of mv_paged_decode_write, in its order. */
static PyObject* decode_write(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (check_nargs("decode_write", n, 35, (const void*)g_decode_write)) return NULL;
  const void* query = arg_ptr(a[0]);
  const int64_t q_st = arg_i64(a[1]), q_sh = arg_i64(a[2]);
  const void* nk = arg_ptr(a[3]);
  const int64_t nk_st = arg_i64(a[4]), nk_sh = arg_i64(a[5]);
  const void* nv = arg_ptr(a[6]);
  const int64_t nv_st = arg_i64(a[7]), nv_sh = arg_i64(a[8]);
  const int64_t* slots = (const int64_t*)arg_ptr(a[9]);
  const void* rope_cos = arg_ptr(a[10]);
  const void* rope_sin = arg_ptr(a[11]);
  void* key_cache = arg_ptr(a[12]);
  void* value_cache = arg_ptr(a[13]);
  const int32_t* work = (const int32_t*)arg_ptr(a[14]);
  const int32_t* ids = (const int32_t*)arg_ptr(a[15]);
  const int64_t ids_cap = arg_i64(a[16]);
  const int32_t groups = arg_i32(a[17]), part_tokens = arg_i32(a[18]), max_parts = arg_i32(a[19]);
  int32_t* counters = (int32_t*)arg_ptr(a[20]);
  void* out = arg_ptr(a[21]);
  const int64_t o_st = arg_i64(a[22]), o_sh = arg_i64(a[23]);
  const float scale = arg_f32(a[24]);
  const int32_t num_seqs = arg_i32(a[25]), hq = arg_i32(a[26]), hkv = arg_i32(a[27]);
  const int32_t d = arg_i32(a[28]), bs = arg_i32(a[29]);
  const int64_t num_blocks = arg_i64(a[30]);
  const int32_t dtype = arg_i32(a[31]);
  void* ws = arg_ptr(a[32]);
  const size_t ws_bytes = arg_size(a[33]);
  void* stream = arg_ptr(a[34]);
  if (PyErr_Occurred()) return NULL;
  const int rc = g_decode_write(query, q_st, q_sh, nk, nk_st, nk_sh, nv, nv_st, nv_sh, slots,
                                rope_cos, rope_sin, key_cache, value_cache, work, ids, ids_cap,
                                groups, part_tokens, max_parts, counters, out, o_st, o_sh, scale,
                                num_seqs, hq, hkv, d, bs, num_blocks, dtype, ws, ws_bytes, stream);
  return PyLong_FromLong(rc);
}

/* The step words of decode_write_step: the arguments of
 * mv_paged_decode_write that do not change between the layers of a step,
 * in its order, each as one little-endian 64-bit word (scale as a double). */
enum {
  SW_SLOTS, SW_ROPE_COS, SW_ROPE_SIN, SW_WORK, SW_IDS, SW_IDS_CAP, SW_GROUPS, SW_PART_TOKENS,
  SW_MAX_PARTS, SW_COUNTERS, SW_SCALE, SW_NUM_SEQS, SW_HQ, SW_HKV, SW_D, SW_BS, SW_NUM_BLOCKS,
  SW_DTYPE, SW_WS, SW_WS_BYTES, STEP_WORDS
};

static int step_i32(const int64_t* w, int i, int32_t* out) {
  if (w[i] < INT32_MIN || w[i] > INT32_MAX) {
    PyErr_Format(PyExc_OverflowError, "_mvlaunch.decode_write_step: step word %d does not fit int32", i);
    return -1;
  }
  *out = (int32_t)w[i];
  return 0;
}

/* decode_write_step(step, query, q_st, q_sh, nk, nk_st, nk_sh, nv, nv_st,
 * nv_sh, key_cache, value_cache, out, o_st, o_sh, stream):
 * mv_paged_decode_write with the step's words and this layer's tensors. */
static PyObject* decode_write_step(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (check_nargs("decode_write_step", n, 16, (const void*)g_decode_write)) return NULL;
  if (!PyBytes_Check(a[0]) || PyBytes_GET_SIZE(a[0]) != (Py_ssize_t)(STEP_WORDS * sizeof(int64_t))) {
    PyErr_SetString(PyExc_TypeError, "_mvlaunch.decode_write_step: step must be bytes of STEP_WORDS words");
    return NULL;
  }
  int64_t w[STEP_WORDS];
  memcpy(w, PyBytes_AS_STRING(a[0]), sizeof w);
  double scale;
  memcpy(&scale, &w[SW_SCALE], sizeof scale);
  int32_t groups, part_tokens, max_parts, num_seqs, hq, hkv, d, bs, dtype;
  if (step_i32(w, SW_GROUPS, &groups) || step_i32(w, SW_PART_TOKENS, &part_tokens) ||
      step_i32(w, SW_MAX_PARTS, &max_parts) || step_i32(w, SW_NUM_SEQS, &num_seqs) ||
      step_i32(w, SW_HQ, &hq) || step_i32(w, SW_HKV, &hkv) || step_i32(w, SW_D, &d) ||
      step_i32(w, SW_BS, &bs) || step_i32(w, SW_DTYPE, &dtype))
    return NULL;
  const void* query = arg_ptr(a[1]);
  const int64_t q_st = arg_i64(a[2]), q_sh = arg_i64(a[3]);
  const void* nk = arg_ptr(a[4]);
  const int64_t nk_st = arg_i64(a[5]), nk_sh = arg_i64(a[6]);
  const void* nv = arg_ptr(a[7]);
  const int64_t nv_st = arg_i64(a[8]), nv_sh = arg_i64(a[9]);
  void* key_cache = arg_ptr(a[10]);
  void* value_cache = arg_ptr(a[11]);
  void* out = arg_ptr(a[12]);
  const int64_t o_st = arg_i64(a[13]), o_sh = arg_i64(a[14]);
  void* stream = arg_ptr(a[15]);
  if (PyErr_Occurred()) return NULL;
  const int rc = g_decode_write(
      query, q_st, q_sh, nk, nk_st, nk_sh, nv, nv_st, nv_sh, (const int64_t*)(intptr_t)w[SW_SLOTS],
      (const void*)(intptr_t)w[SW_ROPE_COS], (const void*)(intptr_t)w[SW_ROPE_SIN], key_cache,
      value_cache, (const int32_t*)(intptr_t)w[SW_WORK], (const int32_t*)(intptr_t)w[SW_IDS],
      w[SW_IDS_CAP], groups, part_tokens, max_parts, (int32_t*)(intptr_t)w[SW_COUNTERS], out, o_st,
      o_sh, (float)scale, num_seqs, hq, hkv, d, bs, w[SW_NUM_BLOCKS], dtype,
      (void*)(intptr_t)w[SW_WS], (size_t)w[SW_WS_BYTES], stream);
  return PyLong_FromLong(rc);
}

/* Arguments of mv_paged_decode, in its order. */
static PyObject* decode(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (check_nargs("decode", n, 26, (const void*)g_decode)) return NULL;
  const void* query = arg_ptr(a[0]);
  const int64_t q_st = arg_i64(a[1]), q_sh = arg_i64(a[2]);
  const void* key_cache = arg_ptr(a[3]);
  const void* value_cache = arg_ptr(a[4]);
  const int32_t* work = (const int32_t*)arg_ptr(a[5]);
  const int32_t* ids = (const int32_t*)arg_ptr(a[6]);
  const int64_t ids_cap = arg_i64(a[7]);
  const int32_t groups = arg_i32(a[8]), part_tokens = arg_i32(a[9]), max_parts = arg_i32(a[10]);
  int32_t* counters = (int32_t*)arg_ptr(a[11]);
  void* out = arg_ptr(a[12]);
  const int64_t o_st = arg_i64(a[13]), o_sh = arg_i64(a[14]);
  const float scale = arg_f32(a[15]);
  const int32_t num_seqs = arg_i32(a[16]), hq = arg_i32(a[17]), hkv = arg_i32(a[18]);
  const int32_t d = arg_i32(a[19]), bs = arg_i32(a[20]);
  const int64_t num_blocks = arg_i64(a[21]);
  const int32_t dtype = arg_i32(a[22]);
  void* ws = arg_ptr(a[23]);
  const size_t ws_bytes = arg_size(a[24]);
  void* stream = arg_ptr(a[25]);
  if (PyErr_Occurred()) return NULL;
  const int rc = g_decode(query, q_st, q_sh, key_cache, value_cache, work, ids, ids_cap, groups,
                          part_tokens, max_parts, counters, out, o_st, o_sh, scale, num_seqs, hq,
                          hkv, d, bs, num_blocks, dtype, ws, ws_bytes, stream);
  return PyLong_FromLong(rc);
}

/* Arguments of mv_kv_cache_write, in its order. */
static PyObject* cache_write(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (check_nargs("cache_write", n, 16, (const void*)g_cache_write)) return NULL;
  const void* key = arg_ptr(a[0]);
  const int64_t k_st = arg_i64(a[1]), k_sh = arg_i64(a[2]);
  const void* value = arg_ptr(a[3]);
  const int64_t v_st = arg_i64(a[4]), v_sh = arg_i64(a[5]);
  void* key_cache = arg_ptr(a[6]);
  void* value_cache = arg_ptr(a[7]);
  const int64_t* slots = (const int64_t*)arg_ptr(a[8]);
  const int64_t num_tokens = arg_i64(a[9]);
  const int32_t hkv = arg_i32(a[10]), d = arg_i32(a[11]), bs = arg_i32(a[12]);
  const int64_t num_blocks = arg_i64(a[13]);
  const int32_t dtype = arg_i32(a[14]);
  void* stream = arg_ptr(a[15]);
  if (PyErr_Occurred()) return NULL;
  const int rc = g_cache_write(key, k_st, k_sh, value, v_st, v_sh, key_cache, value_cache, slots,
                               num_tokens, hkv, d, bs, num_blocks, dtype, stream);
  return PyLong_FromLong(rc);
}

/* Arguments of mv_rope_kv_cache_write, in its order. */
static PyObject* rope_write(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (check_nargs("rope_write", n, 31, (const void*)g_rope_write)) return NULL;
  const void* query = arg_ptr(a[0]);
  const int64_t q_st = arg_i64(a[1]), q_sh = arg_i64(a[2]);
  void* query_out = arg_ptr(a[3]);
  const int64_t qo_st = arg_i64(a[4]), qo_sh = arg_i64(a[5]);
  const void* key = arg_ptr(a[6]);
  const int64_t k_st = arg_i64(a[7]), k_sh = arg_i64(a[8]);
  void* key_out = arg_ptr(a[9]);
  const int64_t ko_st = arg_i64(a[10]), ko_sh = arg_i64(a[11]);
  const void* value = arg_ptr(a[12]);
  const int64_t v_st = arg_i64(a[13]), v_sh = arg_i64(a[14]);
  void* key_cache = arg_ptr(a[15]);
  void* value_cache = arg_ptr(a[16]);
  const int64_t* slots = (const int64_t*)arg_ptr(a[17]);
  const int64_t* positions = (const int64_t*)arg_ptr(a[18]);
  const void* cos_table = arg_ptr(a[19]);
  const void* sin_table = arg_ptr(a[20]);
  const int64_t table_stride = arg_i64(a[21]), max_positions = arg_i64(a[22]);
  const int64_t num_tokens = arg_i64(a[23]);
  const int32_t hq = arg_i32(a[24]), hkv = arg_i32(a[25]), d = arg_i32(a[26]), bs = arg_i32(a[27]);
  const int64_t num_blocks = arg_i64(a[28]);
  const int32_t dtype = arg_i32(a[29]);
  void* stream = arg_ptr(a[30]);
  if (PyErr_Occurred()) return NULL;
  const int rc = g_rope_write(query, q_st, q_sh, query_out, qo_st, qo_sh, key, k_st, k_sh, key_out,
                              ko_st, ko_sh, value, v_st, v_sh, key_cache, value_cache, slots,
                              positions, cos_table, sin_table, table_stride, max_positions,
                              num_tokens, hq, hkv, d, bs, num_blocks, dtype, stream);
  return PyLong_FromLong(rc);
}

/* Arguments of mv_decode_plan, in its order. */
static PyObject* plan(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (check_nargs("plan", n, 20, (const void*)g_plan)) return NULL;
  const void* kv_len = arg_ptr(a[0]);
  const int32_t kv_i64 = arg_i32(a[1]);
  const void* block_table = arg_ptr(a[2]);
  const int32_t bt_i64 = arg_i32(a[3]);
  const int64_t bt_stride = arg_i64(a[4]);
  const int32_t num_seqs = arg_i32(a[5]), max_blocks = arg_i32(a[6]), bs = arg_i32(a[7]);
  const int64_t num_blocks = arg_i64(a[8]);
  const int32_t hkv = arg_i32(a[9]), per_cu = arg_i32(a[10]), cus = arg_i32(a[11]);
  const int32_t fixed = arg_i32(a[12]);
  int32_t* work = (int32_t*)arg_ptr(a[13]);
  const int64_t work_cap = arg_i64(a[14]);
  int32_t* ids = (int32_t*)arg_ptr(a[15]);
  const int64_t ids_cap = arg_i64(a[16]);
  int32_t* counters = (int32_t*)arg_ptr(a[17]);
  int32_t* status = (int32_t*)arg_ptr(a[18]);
  void* stream = arg_ptr(a[19]);
  if (PyErr_Occurred()) return NULL;
  const int rc = g_plan(kv_len, kv_i64, block_table, bt_i64, bt_stride, num_seqs, max_blocks, bs,
                        num_blocks, hkv, per_cu, cus, fixed, work, work_cap, ids, ids_cap,
                        counters, status, stream);
  return PyLong_FromLong(rc);
}

/* bind(decode_write, decode, cache_write, rope_write, plan): the entry
 * points' addresses in the loaded libmvattn.so (ctypes resolves them). */
static PyObject* bind(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (n != 5) {
    PyErr_SetString(PyExc_TypeError, "_mvlaunch.bind takes 5 addresses");
    return NULL;
  }
  void* p[5];
  for (int i = 0; i < 5; ++i) {
    p[i] = PyLong_AsVoidPtr(a[i]);
    if (PyErr_Occurred()) return NULL;
    if (!p[i]) {
      PyErr_SetString(PyExc_ValueError, "_mvlaunch.bind: null address");
      return NULL;
    }
  }
  g_decode_write = (decode_write_fn)p[0];
  g_decode = (decode_fn)p[1];
  g_cache_write = (cache_write_fn)p[2];
  g_rope_write = (rope_write_fn)p[3];
  g_plan = (plan_fn)p[4];
  Py_RETURN_NONE;
}

static PyMethodDef methods[] = {
    {"bind", (PyCFunction)(void (*)(void))bind, METH_FASTCALL, "bind the entry points"},
    {"decode_write", (PyCFunction)(void (*)(void))decode_write, METH_FASTCALL,
     "mv_paged_decode_write with its 35 arguments"},
    {"decode_write_step", (PyCFunction)(void (*)(void))decode_write_step, METH_FASTCALL,
     "mv_paged_decode_write from a step's packed words and one layer's 15 arguments"},
    {"decode", (PyCFunction)(void (*)(void))decode, METH_FASTCALL,
     "mv_paged_decode with its 26 arguments"},
    {"cache_write", (PyCFunction)(void (*)(void))cache_write, METH_FASTCALL,
     "mv_kv_cache_write with its 16 arguments"},
    {"rope_write", (PyCFunction)(void (*)(void))rope_write, METH_FASTCALL,
     "mv_rope_kv_cache_write with its 31 arguments"},
    {"plan", (PyCFunction)(void (*)(void))plan, METH_FASTCALL,
     "mv_decode_plan with its 20 arguments"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_mvlaunch",
                                    "fast-call wrappers of libmvattn entry points", -1, methods,
                                    NULL, NULL, NULL, NULL};

/* The module carries the ABI version of the header it was built against
 * (ABI): the Python side binds it only to a library of the same version. */
PyMODINIT_FUNC PyInit__mvlaunch(void) {
  PyObject* m = PyModule_Create(&module);
  if (m && (PyModule_AddIntConstant(m, "ABI", MVATTN_ABI_VERSION) < 0 ||
            PyModule_AddIntConstant(m, "STEP_WORDS", STEP_WORDS) < 0)) {
    Py_DECREF(m);
    return NULL;
  }
  return m;
}
