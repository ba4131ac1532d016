/* rad_planes.h -- radiance's joined-planes weight blob ("rad.planes"), as the reference's
 * rows and tools read and write it: RECONSTRUCTED.  radiance v1.11.0's own rad_planes.h
 * is not available offline; what is fixed here is what the reference's call sites use:
 *   readers   rad_planes_header(blob), header->n_planes / ->transform[] / ->bytes,
 *             rad_planes_find(blob, role, &entry) and the entry's dtype, block[2], rows,
 *             cols, row_bytes, offset (src/r3d_gemm_logits.hip:176-186,
 *             src/r3d_logit_rerank_e4m3.hip:265-290, src/r3d_gemm_w2a8.hip:1011-1017);
 *   writers   a zeroed blob with the header at byte 0 (magic, n_planes, transform[0],
 *             bytes set), the entry array right after sizeof(RadPlanesHeader), each entry
 *             {role, dtype, kind = RAD_PLANE_TILED, block, rows, cols, row_bytes, offset},
 *             the first plane at rad_planes_round(sizeof header + n * sizeof entry) and
 *             each next one at rad_planes_round(previous offset + its bytes), the blob
 *             ending at the last plane's end (tools/bench_skinny.cpp:206-220,
 *             tools/bench_w2a8.cpp:85-99, tools/repro_w2a8.hip:102-116);
 *   hooks     rad_planes_layout / _relayout / _unrelayout(enc, sel, planes, n, ...), the
 *             canonical join a row's weight-layout hooks answer with
 *             (src/r3d_gemm_logits.hip:253-271, src/r3d_gemm_w2a8.hip:1400-1435).
 * Not recoverable from the reference, and this header's own: the magic value, the width
 * and order of the fields, the role's fixed size, RAD_PLANES_MAX and the rounding unit of
 * rad_planes_round.  The dependency is isolated here so the real header can replace this
 * file without touching any other source.
 */
#ifndef RAD_PLANES_H
#define RAD_PLANES_H

#include <stdint.h>
#include <string.h>

#include "rad_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define RAD_PLANES_MAGIC 0x534E4C50u       /* "PLNS" */
#define RAD_PLANES_MAX 4
#define RAD_PLANES_ROLE 16
#define RAD_PLANES_ALIGN 256
#define RAD_PLANES_TAG "rad.planes"

typedef struct RadPlanesHeader {
    uint32_t magic;                       /* RAD_PLANES_MAGIC */
    uint32_t n_planes;                    /* entries that follow the header */
    uint32_t transform[RAD_PLANES_MAX];   /* [0] non-zero: a rotated encoding */
    int64_t  bytes;                       /* the whole blob, header included */
} RadPlanesHeader;

typedef struct RadPlanesEntry {
    char     role[RAD_PLANES_ROLE];       /* "codes", "scale", ... NUL-padded */
    uint32_t dtype;                       /* RadDtype of one element */
    uint32_t kind;                        /* RadPlaneKind */
    int64_t  block[2];                    /* weight rows x cols one element covers */
    int64_t  rows, cols;                  /* the element grid */
    int64_t  row_bytes;                   /* pitch of the grid's rows */
    int64_t  offset;                      /* first byte, from the blob's start */
} RadPlanesEntry;

/* The start of a blob up to its last possible entry: what a host copy of a header holds. */
typedef struct RadPlanesHead {
    RadPlanesHeader h;
    RadPlanesEntry  e[RAD_PLANES_MAX];
} RadPlanesHead;

static inline int64_t rad_planes_round(int64_t v) {
    return (v + RAD_PLANES_ALIGN - 1) / RAD_PLANES_ALIGN * RAD_PLANES_ALIGN;
}

static inline const RadPlanesEntry* rad_planes_entries(const RadPlanesHeader* h) {
    return (const RadPlanesEntry*)(h + 1);
}

/* The header at the start of a blob (host-readable memory), or null without one. */
static inline const RadPlanesHeader* rad_planes_header(const void* blob) {
    const RadPlanesHeader* h = (const RadPlanesHeader*)blob;
    if (!h || h->magic != RAD_PLANES_MAGIC || h->n_planes < 1 || h->n_planes > RAD_PLANES_MAX)
        return 0;
    return h;
}

/* The plane of role `role` in the blob whose header (and entries) `h` points at -- the blob
 * itself or a host copy of its start -- or null; *e (if given) receives its entry.  The
 * returned address is `base` + the entry's offset, so it points into whichever copy of the
 * blob `base` addresses. */
static inline const void* rad_planes_find_at(const RadPlanesHeader* h, const void* base,
                                            const char* role, const RadPlanesEntry** e) {
    if (!h) return 0;
    const RadPlanesEntry* en = rad_planes_entries(h);
    for (uint32_t i = 0; i < h->n_planes; ++i)
        if (strncmp(en[i].role, role, RAD_PLANES_ROLE) == 0) {
            if (e) *e = &en[i];
            /* address arithmetic on integers: an offset the reader has not validated yet
             * (the plan checks it against the blob's extent) cannot overflow a pointer */
            return (const void*)((uintptr_t)base + (uint64_t)en[i].offset);
        }
    return 0;
}

static inline const void* rad_planes_find(const void* blob, const char* role,
                                          const RadPlanesEntry** e) {
    return rad_planes_find_at(rad_planes_header(blob), blob, role, e);
}

/* ---- the canonical join behind a row's layout hooks ---------------------------------- */

/* Bits of one element of dtype (0: not a plane dtype). */
static inline int rad_planes_elem_bits(uint32_t dtype) {
    switch (dtype) {
    case RAD_F32: case RAD_I32: case RAD_U32: return 32;
    case RAD_BF16: case RAD_F16: case RAD_I16: return 16;
    case RAD_F8E4M3: case RAD_F8E5M2: case RAD_E8M0: case RAD_U8: case RAD_I8: case RAD_BOOL:
        return 8;
    case RAD_FP4E2M1: case RAD_U4: return 4;
    case RAD_U2: return 2;
    case RAD_I64: return 64;
    default: return 0;
    }
}

/* The largest row count, column count or row pitch (elements) a plane may have here. */
#define RAD_PLANES_DIM_MAX ((int64_t)1 << 28)

/* A plane tensor's element grid (rank 1: one row; rank 2: rows x cols, inner stride 1)
 * and its row pitch in elements; RAD_OK or the refusal. */
static inline int rad_planes_grid(const RadTensor* t, int64_t* rows, int64_t* cols,
                                  int64_t* pitch) {
    if (t->rank == 1) {
        *rows = 1;
        *cols = t->shape[0];
        *pitch = t->shape[0];
    } else if (t->rank == 2) {
        if (t->stride[1] != 1) return RAD_E_STRIDE;
        *rows = t->shape[0];
        *cols = t->shape[1];
        *pitch = t->stride[0];
    } else {
        return RAD_E_SHAPE;
    }
    if (*rows <= 0 || *cols <= 0 || *pitch < *cols) return RAD_E_SHAPE;
    /* extents whose products (rows x row bytes, pitch x bits) stay far inside int64 */
    if (*rows > RAD_PLANES_DIM_MAX || *pitch > RAD_PLANES_DIM_MAX) return RAD_E_SHAPE;
    return RAD_OK;
}

/* The joined blob for planes[0..n) (planes[i] holding encoding plane sel[i]): header and
 * entries into *head (when given), its size in *bytes.  Rows are stored dense. */
static inline int rad_planes_plan(const RadEncoding* enc, const int* sel,
                                  const RadTensor* planes, int n, RadPlanesHead* head,
                                  int64_t* bytes) {
    if (!enc || !sel || !planes || n < 1 || n > RAD_PLANES_MAX) return RAD_E_INVAL;
    RadPlanesHead hd;
    memset(&hd, 0, sizeof hd);
    hd.h.magic = RAD_PLANES_MAGIC;
    hd.h.n_planes = (uint32_t)n;
    for (int i = 0; i < RAD_PLANES_MAX && i < RAD_ENC_MAX_PLANES; ++i)
        hd.h.transform[i] = enc->transform[i];
    int64_t off = rad_planes_round((int64_t)(sizeof(RadPlanesHeader) +
                                             (size_t)n * sizeof(RadPlanesEntry)));
    int64_t end = off;
    for (int i = 0; i < n; ++i) {
        if (sel[i] < 0 || sel[i] >= enc->n_planes || sel[i] >= RAD_ENC_MAX_PLANES)
            return RAD_E_DTYPE;
        const RadEncPlane* ep = &enc->plane[sel[i]];
        const int bits = rad_planes_elem_bits(ep->dtype);
        if (!bits || planes[i].dtype != ep->dtype) return RAD_E_DTYPE;
        int64_t rows = 0, cols = 0, pitch = 0;
        const int rc = rad_planes_grid(&planes[i], &rows, &cols, &pitch);
        if (rc) return rc;
        RadPlanesEntry* e = &hd.e[i];
        memcpy(e->role, ep->role, RAD_PLANES_ROLE < RAD_ENC_STR ? RAD_PLANES_ROLE : RAD_ENC_STR);
        e->dtype = ep->dtype;
        e->kind = ep->kind;
        e->block[0] = ep->block[0];
        e->block[1] = ep->block[1];
        e->rows = rows;
        e->cols = cols;
        e->row_bytes = (cols * bits + 7) / 8;
        if (i) off = rad_planes_round(end);
        e->offset = off;
        end = off + rows * e->row_bytes;
    }
    hd.h.bytes = end;
    if (head) *head = hd;
    if (bytes) *bytes = end;
    return RAD_OK;
}

static inline int rad_planes_layout(const RadEncoding* enc, const int* sel,
                                    const RadTensor* planes, int n, RadLayout* out) {
    int64_t bytes = 0;
    const int rc = rad_planes_plan(enc, sel, planes, n, 0, &bytes);
    if (rc) return rc;
    if (out) {
        out->tag = RAD_PLANES_TAG;
        out->bytes = bytes;
    }
    return RAD_OK;
}

/* Writes the joined blob into host memory dst: every plane's data must be present (at
 * declare time the planes carry geometry only). */
static inline int rad_planes_relayout(const RadEncoding* enc, const int* sel,
                                      const RadTensor* planes, int n, void* dst,
                                      int64_t dst_bytes) {
    RadPlanesHead hd;
    int64_t bytes = 0;
    const int rc = rad_planes_plan(enc, sel, planes, n, &hd, &bytes);
    if (rc) return rc;
    if (!dst || dst_bytes < bytes) return RAD_E_SHAPE;
    for (int i = 0; i < n; ++i)
        if (!planes[i].data) return RAD_E_INVAL;
    uint8_t* d = (uint8_t*)dst;
    memset(d, 0, (size_t)bytes);
    memcpy(d, &hd.h, sizeof hd.h);
    memcpy(d + sizeof hd.h, hd.e, (size_t)n * sizeof(RadPlanesEntry));
    for (int i = 0; i < n; ++i) {
        const RadPlanesEntry* e = &hd.e[i];
        int64_t rows = 0, cols = 0, pitch = 0;
        rad_planes_grid(&planes[i], &rows, &cols, &pitch);
        const int bits = rad_planes_elem_bits(e->dtype);
        if ((pitch * bits) % 8) return RAD_E_STRIDE;      /* sub-byte rows start on a byte */
        const int64_t src_pitch = pitch * bits / 8;
        for (int64_t r = 0; r < rows; ++r)
            memcpy(d + e->offset + r * e->row_bytes,
                   (const uint8_t*)planes[i].data + r * src_pitch, (size_t)e->row_bytes);
    }
    return RAD_OK;
}

/* Reads the planes back out of a joined blob in host memory (found by their encoding
 * roles, which must carry the planes' dtypes and grids). */
static inline int rad_planes_unrelayout(const RadEncoding* enc, const int* sel, const void* src,
                                        int64_t src_bytes, const RadTensor* planes, int n) {
    if (!enc || !sel || !planes || n < 1 || n > RAD_PLANES_MAX) return RAD_E_INVAL;
    if (!src || src_bytes < (int64_t)sizeof(RadPlanesHeader)) return RAD_E_SHAPE;
    const RadPlanesHeader* h = rad_planes_header(src);
    if (!h) return RAD_E_DTYPE;
    if ((int64_t)(sizeof(RadPlanesHeader) + h->n_planes * sizeof(RadPlanesEntry)) > src_bytes ||
        h->bytes > src_bytes)
        return RAD_E_SHAPE;
    for (int i = 0; i < n; ++i) {
        if (sel[i] < 0 || sel[i] >= enc->n_planes || sel[i] >= RAD_ENC_MAX_PLANES)
            return RAD_E_DTYPE;
        char role[RAD_PLANES_ROLE + 1];
        memset(role, 0, sizeof role);
        memcpy(role, enc->plane[sel[i]].role,
               RAD_PLANES_ROLE < RAD_ENC_STR ? RAD_PLANES_ROLE : RAD_ENC_STR);
        const RadPlanesEntry* e = 0;
        if (!rad_planes_find(src, role, &e) || !e) return RAD_E_DTYPE;
        if (e->dtype != planes[i].dtype) return RAD_E_DTYPE;
        const int bits = rad_planes_elem_bits(e->dtype);
        int64_t rows = 0, cols = 0, pitch = 0;
        const int rc = rad_planes_grid(&planes[i], &rows, &cols, &pitch);
        if (rc) return rc;
        const int64_t need = (cols * bits + 7) / 8;
        if (e->rows != rows || e->cols != cols || e->row_bytes < need) return RAD_E_SHAPE;
        int64_t span = 0, end = 0;                 /* the header's own fields: checked sums */
        if (e->offset < 0 || __builtin_mul_overflow(rows, e->row_bytes, &span) ||
            __builtin_add_overflow(e->offset, span, &end) || end > h->bytes)
            return RAD_E_SHAPE;
        if ((pitch * bits) % 8) return RAD_E_STRIDE;
        if (!planes[i].data) return RAD_E_INVAL;
        for (int64_t r = 0; r < rows; ++r)
            memcpy((uint8_t*)planes[i].data + r * (pitch * bits / 8),
                   (const uint8_t*)src + e->offset + r * e->row_bytes, (size_t)need);
    }
    return RAD_OK;
}

#ifdef __cplusplus
}
#endif

#endif /* RAD_PLANES_H */
