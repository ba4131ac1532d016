/* r3d_head.cpp -- the joined e4m3 lm_head on the host: the logits_gemm_e4m3 row's weight-
 * layout hooks (the reference's r3d_layout_head / r3d_relayout_head / r3d_unrelayout_head,
 * src/r3d_gemm_logits.hip:230-272, registered at src/r3d_rows.cpp:1598-1599) and this
 * library's own join / split calls, which write and read the same blob.  Host only: no
 * device memory is touched here.
 */
#include <string.h>

#include "r3d_gfx950.h"
#include "r3d_plan.h"
#include "rad_planes.h"
#include "rad_plugin.h"

namespace r3d {

static bool scale_dtype_ok(uint32_t dt) { return dt == RAD_BF16 || dt == RAD_F16 || dt == RAD_F32; }

static bool role_is(const char* role, const char* want) {
    return strncmp(role, want, RAD_ENC_STR) == 0;
}

/* An integer parameter by key, or `fb`. */
static long long param_i(const RadParam* p, int n_p, const char* key, long long fb) {
    for (int i = 0; p && i < n_p; ++i)
        if (p[i].key && strcmp(p[i].key, key) == 0 && p[i].kind == RAD_P_INT) return p[i].ival;
    return fb;
}

/* The hooks' gate.  The reference's, in its order and with its answers
 * (src/r3d_gemm_logits.hip:233-253): an operand other than the head (1) is stored as it
 * is; the selection must be the encoding's two planes "codes" then "scale", of an
 * untransformed "affine" encoding, codes tiled 1 x 1 e4m3 and a tiled bf16 / f16 / f32
 * scale -- anything else declines (RAD_E_DTYPE).
 * Then what this row's launch would refuse, declined here at declare time instead of
 * refused at issue time (an issue-time refusal aborts the engine,
 * src/r3d_rows.cpp:2197-2215): a scale block other than (1 or 128) x 128, n_embd not a
 * multiple of 4 or too long to stage (RAD_E_DTYPE), planes whose grids disagree with each
 * other or with the n_vocab / n_embd parameters (RAD_E_SHAPE).
 * One deliberate difference: the reference answers RAD_E_UNSUPPORTED ("store as is") for
 * a head without the two-plane encoding -- a plain bf16 head -- because its own
 * logits_gemm_bf16 row, declared first, claims such heads (src/r3d_rows.cpp:1570-1585).
 * This library has no bf16 head row, so a plain head is declined here (RAD_E_DTYPE) and
 * resolves past this row instead of being claimed and then refused at launch. */
static int head_gate(const RadParam* p, int n_p, int operand, const RadEncoding* enc,
                     const int* sel, const RadTensor* planes, int n) {
    if (operand != 1) return RAD_E_UNSUPPORTED;
    if (!enc || !sel || !planes || n != 2) return RAD_E_DTYPE;
    for (int i = 0; i < 2; ++i)
        if (sel[i] < 0 || sel[i] >= enc->n_planes || sel[i] >= RAD_ENC_MAX_PLANES)
            return RAD_E_DTYPE;
    if (enc->n_planes != 2 || enc->transform[0]) return RAD_E_DTYPE;
    const RadEncPlane& c = enc->plane[sel[0]];
    const RadEncPlane& sl = enc->plane[sel[1]];
    if (!role_is(c.role, "codes") || !role_is(sl.role, "scale")) return RAD_E_DTYPE;
    if (c.kind != RAD_PLANE_TILED || c.block[0] != 1 || c.block[1] != 1 || c.dtype != RAD_F8E4M3)
        return RAD_E_DTYPE;
    if (sl.kind != RAD_PLANE_TILED || !scale_dtype_ok(sl.dtype)) return RAD_E_DTYPE;
    if (!role_is(enc->scheme, "affine")) return RAD_E_DTYPE;

    /* this row's launch */
    if (sl.block[1] != 128 || (sl.block[0] != 1 && sl.block[0] != 128)) return RAD_E_DTYPE;
    const RadTensor& pc = planes[0];
    const RadTensor& ps = planes[1];
    if (pc.rank != 2 || ps.rank != 2) return RAD_E_SHAPE;
    const int64_t N = pc.shape[0], K = pc.shape[1];
    if (N <= 0 || K <= 0 || N > 0x7FFFFFFLL || K > 0x7FFFFFFLL) return RAD_E_SHAPE;
    if (ps.shape[0] != (N + sl.block[0] - 1) / sl.block[0] || ps.shape[1] != (K + 127) / 128)
        return RAD_E_SHAPE;
    if (param_i(p, n_p, "n_vocab", N) != N || param_i(p, n_p, "n_embd", K) != K) return RAD_E_SHAPE;
    if (K & 3) return RAD_E_DTYPE;
    if (64 * K > 0x7FFFFFFFLL || !logits_shape(1, K, nullptr)) return RAD_E_DTYPE;
    const int64_t ssz = sl.dtype == RAD_F32 ? 4 : 2;
    if (ps.shape[0] * ps.shape[1] * ssz > 0x7FFFFFFFLL) return RAD_E_DTYPE;
    return RAD_OK;
}

/* The encoding and plane tensors of a head the library joins itself. */
static void head_encoding(uint32_t sdt, int64_t br, RadEncoding* enc) {
    memset(enc, 0, sizeof *enc);
    strncpy(enc->scheme, "affine", RAD_ENC_STR);
    enc->n_planes = 2;
    strncpy(enc->plane[0].role, "codes", RAD_ENC_STR);
    enc->plane[0].kind = RAD_PLANE_TILED;
    enc->plane[0].dtype = RAD_F8E4M3;
    enc->plane[0].block[0] = enc->plane[0].block[1] = 1;
    strncpy(enc->plane[1].role, "scale", RAD_ENC_STR);
    enc->plane[1].kind = RAD_PLANE_TILED;
    enc->plane[1].dtype = sdt;
    enc->plane[1].block[0] = br;
    enc->plane[1].block[1] = 128;
}

static void plane_tensor(RadTensor* t, const void* data, uint32_t dtype, int64_t rows,
                         int64_t cols, int64_t pitch) {
    memset(t, 0, sizeof *t);
    t->data = const_cast<void*>(data);
    t->dtype = dtype;
    t->rank = 2;
    t->shape[0] = rows;
    t->shape[1] = cols;
    t->stride[0] = pitch;
    t->stride[1] = 1;
}

/* The joined head's header and size for n_vocab x n_embd codes and a scale plane of sdt
 * with br rows per element: the blob's bytes, or minus a RAD_E_* code. */
static int64_t head_plan(int64_t N, int64_t K, uint32_t sdt, int64_t br, RadPlanesHead* head) {
    if (N <= 0 || K <= 0 || N > 0x7FFFFFFLL || K > 0x7FFFFFFLL) return -RAD_E_SHAPE;
    if (!scale_dtype_ok(sdt)) return -RAD_E_DTYPE;
    if (br != 1 && br != 128) return -RAD_E_SHAPE;
    RadEncoding enc;
    head_encoding(sdt, br, &enc);
    const int sel[2] = {0, 1};
    RadTensor planes[2];
    const int64_t srows = (N + br - 1) / br, scols = (K + 127) / 128;
    plane_tensor(&planes[0], nullptr, RAD_F8E4M3, N, K, K);
    plane_tensor(&planes[1], nullptr, sdt, srows, scols, scols);
    int64_t bytes = 0;
    const int rc = rad_planes_plan(&enc, sel, planes, 2, head, &bytes);
    return rc ? -rc : bytes;
}

}  // namespace r3d

extern "C" {

int r3d_layout_head(const RadParam* p, int n_p, int operand, const RadEncoding* enc,
                    const int* sel, const RadTensor* planes, int n, RadLayout* out) {
    const int rc = r3d::head_gate(p, n_p, operand, enc, sel, planes, n);
    if (rc) return rc;
    return rad_planes_layout(enc, sel, planes, n, out);
}

int r3d_relayout_head(const RadParam* p, int n_p, int operand, const RadEncoding* enc,
                      const int* sel, const RadTensor* planes, int n, void* dst,
                      int64_t dst_bytes) {
    const int rc = r3d::head_gate(p, n_p, operand, enc, sel, planes, n);
    if (rc) return rc;
    return rad_planes_relayout(enc, sel, planes, n, dst, dst_bytes);
}

int r3d_unrelayout_head(const RadParam* p, int n_p, int operand, const RadEncoding* enc,
                        const int* sel, const void* src, int64_t src_bytes,
                        const RadTensor* planes, int n) {
    const int rc = r3d::head_gate(p, n_p, operand, enc, sel, planes, n);
    if (rc) return rc;
    return rad_planes_unrelayout(enc, sel, src, src_bytes, planes, n);
}

int64_t r3d_gfx950_logits_head_bytes(int64_t n_vocab, int64_t n_embd, uint32_t scale_dtype,
                                     int64_t scale_block_rows) {
    return r3d::head_plan(n_vocab, n_embd, scale_dtype, scale_block_rows, nullptr);
}

int64_t r3d_gfx950_logits_head_header(int64_t n_vocab, int64_t n_embd, uint32_t scale_dtype,
                                      int64_t scale_block_rows, RadPlanesHead* out) {
    if (!out) return -RAD_E_INVAL;
    return r3d::head_plan(n_vocab, n_embd, scale_dtype, scale_block_rows, out);
}

int r3d_gfx950_logits_head_join(const uint8_t* codes, int64_t codes_pitch, const void* scale,
                                int64_t scale_pitch_bytes, int64_t n_vocab, int64_t n_embd,
                                uint32_t scale_dtype, int64_t scale_block_rows, void* dst,
                                int64_t dst_bytes) {
    const int64_t need = r3d::head_plan(n_vocab, n_embd, scale_dtype, scale_block_rows, nullptr);
    if (need < 0) return (int)-need;
    if (!codes || !scale || !dst) return RAD_E_INVAL;
    const int64_t esz = scale_dtype == RAD_F32 ? 4 : 2;
    const int64_t srows = (n_vocab + scale_block_rows - 1) / scale_block_rows;
    const int64_t scols = (n_embd + 127) / 128;
    if (codes_pitch < n_embd || scale_pitch_bytes < scols * esz || scale_pitch_bytes % esz)
        return RAD_E_STRIDE;
    RadEncoding enc;
    r3d::head_encoding(scale_dtype, scale_block_rows, &enc);
    const int sel[2] = {0, 1};
    RadTensor planes[2];
    r3d::plane_tensor(&planes[0], codes, RAD_F8E4M3, n_vocab, n_embd, codes_pitch);
    r3d::plane_tensor(&planes[1], scale, scale_dtype, srows, scols, scale_pitch_bytes / esz);
    return rad_planes_relayout(&enc, sel, planes, 2, dst, dst_bytes);
}

int r3d_gfx950_logits_head_split(const void* blob, int64_t blob_bytes, uint8_t* codes,
                                 void* scale) {
    if (!blob || blob_bytes < (int64_t)sizeof(RadPlanesHeader)) return RAD_E_SHAPE;
    const RadPlanesHeader* h = rad_planes_header(blob);
    if (!h) return RAD_E_DTYPE;
    if ((int64_t)(sizeof(RadPlanesHeader) + h->n_planes * sizeof(RadPlanesEntry)) > blob_bytes)
        return RAD_E_SHAPE;
    const RadPlanesEntry* c = nullptr;
    const RadPlanesEntry* e = nullptr;
    if (h->n_planes != 2 || !rad_planes_find(blob, "codes", &c) ||
        !rad_planes_find(blob, "scale", &e))
        return RAD_E_DTYPE;
    if (c->dtype != RAD_F8E4M3 || !r3d::scale_dtype_ok(e->dtype)) return RAD_E_DTYPE;
    if (c->rows <= 0 || c->cols <= 0 || e->rows <= 0 || e->cols <= 0) return RAD_E_SHAPE;
    /* each plane asked for, read back through the same join into a dense host plane (the
     * unrelayout checks its dtype, grid, pitch and extent against the blob) */
    RadEncoding enc;
    r3d::head_encoding(e->dtype, e->block[0], &enc);
    int rc = RAD_OK;
    for (int i = 0; i < 2 && rc == RAD_OK; ++i) {
        void* dst = i == 0 ? (void*)codes : scale;
        if (!dst) continue;
        const RadPlanesEntry* pe = i == 0 ? c : e;
        RadTensor t;
        r3d::plane_tensor(&t, dst, pe->dtype, pe->rows, pe->cols, pe->cols);
        rc = rad_planes_unrelayout(&enc, &i, blob, blob_bytes, &t, 1);
    }
    return rc;
}

}  /* extern "C" */
