/*
 * CPython entry for the public decode call of a shape seen before: the
 * constant arguments of tmla_mla_decode (strides, sizes, element type, scale,
 * split choice, workspace size) are packed once per shape into a capsule
 * (plan), and each call passes only its eight pointers as Python ints
 * (decode, METH_FASTCALL), so the per-call conversion work is eight integers
 * instead of ctypes' twenty-seven typed arguments. The call is made with the
 * GIL held, as the ctypes.PyDLL binding does, so two Python threads on one
 * stream cannot interleave the launches of two calls that share a workspace.
 *
 * Linked against libtriton_mla_hip.so in the same directory (rpath $ORIGIN),
 * the library the ctypes binding loads by the same path.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <stdint.h>

#include "triton_mla.h"

typedef struct {
    int64_t q_sb, q_sh, kv_s0, kv_s1, num_blocks, bt_sb, out_sb, out_sh;
    int32_t page_size, bt_cols, batch, heads, dv, dr, dtype, splits, workers;
    float scale;
    size_t ws_bytes;
} Plan;

static const char kPlanName[] = "triton_mla.plan";

static void plan_free(PyObject* cap) { PyMem_Free(PyCapsule_GetPointer(cap, kPlanName)); }

/* plan(q_sb, q_sh, kv_s0, kv_s1, num_blocks, page_size, bt_sb, bt_cols, batch,
 *      heads, head_dim_v, rope_dim, dtype, scale, num_splits, num_workers,
 *      out_sb, out_sh, ws_bytes) -> capsule */
static PyObject* plan(PyObject* self, PyObject* args) {
    (void)self;
    long long q_sb, q_sh, kv_s0, kv_s1, num_blocks, bt_sb, out_sb, out_sh;
    int page_size, bt_cols, batch, heads, dv, dr, dtype, splits, workers;
    float scale;
    Py_ssize_t ws_bytes;
    if (!PyArg_ParseTuple(args, "LLLLLiLiiiiiifiiLLn", &q_sb, &q_sh, &kv_s0, &kv_s1, &num_blocks, &page_size,
                          &bt_sb, &bt_cols, &batch, &heads, &dv, &dr, &dtype, &scale, &splits, &workers, &out_sb,
                          &out_sh, &ws_bytes))
        return NULL;
    if (ws_bytes < 0) {
        PyErr_SetString(PyExc_ValueError, "ws_bytes must be >= 0");
        return NULL;
    }
    Plan* p = (Plan*)PyMem_Malloc(sizeof(Plan));
    if (p == NULL) return PyErr_NoMemory();
    p->q_sb = q_sb;
    p->q_sh = q_sh;
    p->kv_s0 = kv_s0;
    p->kv_s1 = kv_s1;
    p->num_blocks = num_blocks;
    p->bt_sb = bt_sb;
    p->out_sb = out_sb;
    p->out_sh = out_sh;
    p->page_size = page_size;
    p->bt_cols = bt_cols;
    p->batch = batch;
    p->heads = heads;
    p->dv = dv;
    p->dr = dr;
    p->dtype = dtype;
    p->splits = splits;
    p->workers = workers;
    p->scale = scale;
    p->ws_bytes = (size_t)ws_bytes;
    PyObject* cap = PyCapsule_New(p, kPlanName, plan_free);
    if (cap == NULL) PyMem_Free(p);
    return cap;
}

/* decode(plan, q, kv, block_table, seqlens, out, lse, workspace, stream) ->
 * tmla_status; pointers as ints, None for NULL (block_table, lse). */
static PyObject* decode(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
    (void)self;
    if (nargs != 9) {
        PyErr_SetString(PyExc_TypeError, "decode takes 9 arguments");
        return NULL;
    }
    const Plan* p = (const Plan*)PyCapsule_GetPointer(args[0], kPlanName);
    if (p == NULL) return NULL;
    void* ptr[8];
    for (int i = 0; i < 8; ++i) {
        PyObject* o = args[1 + i];
        if (o == Py_None) {
            ptr[i] = NULL;
        } else {
            ptr[i] = PyLong_AsVoidPtr(o);
            if (ptr[i] == NULL && PyErr_Occurred()) return NULL;
        }
    }
    const int st = tmla_mla_decode(ptr[0], p->q_sb, p->q_sh, ptr[1], p->kv_s0, p->kv_s1, p->num_blocks, p->page_size,
                                   (const int32_t*)ptr[2], p->bt_sb, p->bt_cols, (const int32_t*)ptr[3], p->batch,
                                   p->heads, p->dv, p->dr, p->dtype, p->scale, p->splits, p->workers, ptr[4],
                                   p->out_sb, p->out_sh, (float*)ptr[5], ptr[6], p->ws_bytes, ptr[7]);
    return PyLong_FromLong(st);
}

static PyMethodDef kMethods[] = {
    {"plan", plan, METH_VARARGS, "Pack the constant arguments of tmla_mla_decode for one shape."},
    {"decode", (PyCFunction)(void (*)(void))decode, METH_FASTCALL,
     "tmla_mla_decode(plan, q, kv, block_table, seqlens, out, lse, workspace, stream) -> status."},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_tmla_fast", NULL, -1, kMethods,
                                     NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__tmla_fast(void) { return PyModule_Create(&kModule); }
