// _tmfast: a CPython binding of the per-step op4 greedy path of
// libtreemoe_amd.so.  The ctypes binding converts each argument through a
// Python-level type object (~3.5 us per call of ~18 arguments on the GPU
// host); this module parses them with PyArg_ParseTuple and calls the C ABI
// directly, so one greedy verify + KV commit costs one Python-to-C
// transition.  It adds no semantics: every function here is a plain call of
// the entry points declared in include/treemoe_amd.h.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <stdint.h>

#include "../../include/treemoe_amd.h"

namespace {

// argmax_walk(logits, dtype, N, V, row_stride, tokens, child_start,
//             child_count, child_list, num_edges, max_depth, softmax_argmax,
//             argmax, accepted_slots, accepted_tokens, result, workspace,
//             stream) -> status
PyObject* py_argmax_walk(PyObject*, PyObject* args) {
  unsigned long long logits, tokens, cs, cc, cl, argmax, slots, toks, result, ws, stream;
  int dtype, softmax_argmax;
  long long n, v, row_stride, num_edges, max_depth;
  if (!PyArg_ParseTuple(args, "KiLLLKKKKLLiKKKKKK", &logits, &dtype, &n, &v, &row_stride,
                        &tokens, &cs, &cc, &cl, &num_edges, &max_depth, &softmax_argmax,
                        &argmax, &slots, &toks, &result, &ws, &stream))
    return nullptr;
  const int rc = tm_op4_argmax_walk(
      (const void*)logits, dtype, n, v, row_stride, (const int64_t*)tokens,
      (const int32_t*)cs, (const int32_t*)cc, (const int32_t*)cl, num_edges, max_depth,
      softmax_argmax, (int32_t*)argmax, (int64_t*)slots, (int64_t*)toks, (int64_t*)result,
      (void*)ws, (void*)stream);
  return PyLong_FromLong(rc);
}

// kv_commit(k, v, elem_bytes, L, row_elems, stride_layer, stride_page,
//           stride_slot, page_size, accepted_slots, result, scratch_pages,
//           num_scratch_pages, block_table, num_table_pages, seq_len,
//           max_depth, host_count, stream) -> status
PyObject* py_kv_commit(PyObject*, PyObject* args) {
  unsigned long long k, vv, slots, result, scratch, table, host_count, stream;
  long long elem, layers, row_elems, sl, sp, ss, page, n_scratch, n_table, seq_len, depth;
  if (!PyArg_ParseTuple(args, "KKLLLLLLLKKKLKLLLKK", &k, &vv, &elem, &layers, &row_elems, &sl,
                        &sp, &ss, &page, &slots, &result, &scratch, &n_scratch, &table,
                        &n_table, &seq_len, &depth, &host_count, &stream))
    return nullptr;
  const int rc = tm_op4_kv_commit((void*)k, (void*)vv, elem, layers, row_elems, sl, sp, ss, page,
                                  (const int64_t*)slots, (const int64_t*)result,
                                  (const int32_t*)scratch, n_scratch, (const int32_t*)table,
                                  n_table, seq_len, depth, (int64_t*)host_count, (void*)stream);
  return PyLong_FromLong(rc);
}

PyMethodDef kMethods[] = {
    {"argmax_walk", py_argmax_walk, METH_VARARGS, "tm_op4_argmax_walk"},
    {"kv_commit", py_kv_commit, METH_VARARGS, "tm_op4_kv_commit"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_tmfast", "CPython calls of libtreemoe_amd.so",
                       -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__tmfast(void) { return PyModule_Create(&kModule); }
