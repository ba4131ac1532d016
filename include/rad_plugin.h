/* rad_plugin.h -- host-side argument helpers a radiance kernel row uses, reconstructed
 * from their call sites in the reference (rad_arg_in: src/r3d_gemm_mxfp4.hip:1594-1600;
 * rad_args_geti / rad_args_gets: :1523-1529; rad_tensor_numel: :1536).  Semantics:
 *   rad_arg_in(a, i)      the i-th operand, or null when absent (index past n_t, null
 *                         data pointer, or a rank past RAD_MAX_RANK);
 *   rad_args_geti/gets    look a parameter up by key, 1 when found with that kind;
 *   rad_args_getf_or      an F64 parameter by key, else the fallback;
 *   rad_tensor_numel      product of the shape (0 for a null tensor, -1 for a negative
 *                         extent or an int64 overflow).
 */
#ifndef RAD_PLUGIN_H
#define RAD_PLUGIN_H

#include <string.h>
#include "rad_abi.h"

static inline const RadTensor* rad_arg_in(const RadArgs* a, int i) {
    if (!a || i < 0 || i >= a->n_t || !a->t) return 0;
    /* a rank past RAD_MAX_RANK has no shape to read: treated as absent (refused by every
     * row that needs the operand) */
    return a->t[i].data && a->t[i].rank <= RAD_MAX_RANK ? &a->t[i] : 0;
}

static inline int rad_args_geti(const RadArgs* a, const char* key, long long* out) {
    if (!a || !a->p) return 0;
    for (int i = 0; i < a->n_p; ++i)
        if (a->p[i].key && strcmp(a->p[i].key, key) == 0 && a->p[i].kind == RAD_P_INT) {
            *out = a->p[i].ival;
            return 1;
        }
    return 0;
}

static inline const char* rad_args_gets(const RadArgs* a, const char* key) {
    if (!a || !a->p) return 0;
    for (int i = 0; i < a->n_p; ++i)
        if (a->p[i].key && strcmp(a->p[i].key, key) == 0 && a->p[i].kind == RAD_P_STR)
            return a->p[i].sval;
    return 0;
}

/* A float parameter by key, or `fb` when absent or not an F64 (call sites
 * src/r3d_band.hip:565, src/r3d_more.hip:361). */
static inline double rad_args_getf_or(const RadArgs* a, const char* key, double fb) {
    if (!a || !a->p) return fb;
    for (int i = 0; i < a->n_p; ++i)
        if (a->p[i].key && strcmp(a->p[i].key, key) == 0 && a->p[i].kind == RAD_P_F64)
            return a->p[i].dval;
    return fb;
}

/* Elements of t (the product of its shape); -1 for a negative extent or a product past
 * int64, which every caller's size check then refuses. */
static inline long long rad_tensor_numel(const RadTensor* t) {
    if (!t) return 0;
    long long n = 1;
    for (uint32_t i = 0; i < t->rank && i < RAD_MAX_RANK; ++i) {
        if (t->shape[i] < 0 || __builtin_mul_overflow(n, (long long)t->shape[i], &n)) return -1;
    }
    return n;
}

#endif /* RAD_PLUGIN_H */
