/* rad_planes.h -- radiance's joined-planes weight blob, as the reference's rows read it:
 * RECONSTRUCTED.  radiance v1.11.0's own rad_planes.h is not available offline; what is
 * fixed here is what the reference's call sites use (src/r3d_gemm_logits.hip:159-177,
 * src/r3d_logit_rerank_e4m3.hip:265-290, src/r3d_gemm_w2a8.hip:1011-1016):
 *   rad_planes_header(blob)          the header, or null when the blob carries none;
 *   header->n_planes, ->transform[], ->bytes (the whole blob);
 *   rad_planes_find(blob, role, &e)  the plane whose role is `role` ("codes", "scale",
 *                                    "zero"): its entry and its first byte;
 *   entry->dtype, ->block[2] (rows x cols of the weight one element covers), ->rows,
 *   ->cols (the element grid), ->row_bytes (pitch), ->offset (from the blob's start).
 * The byte layout -- magic, field widths and order, the role's fixed-size name -- is this
 * header's own and could not be checked against radiance's; it is isolated here so the
 * real header can replace this file without touching any other source.
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
#define RAD_PLANES_VERSION 1u
#define RAD_PLANES_MAX 4
#define RAD_PLANES_ROLE 16

typedef struct RadPlanesEntry {
    char     role[RAD_PLANES_ROLE];       /* "codes", "scale", ... NUL-padded */
    uint32_t dtype;                       /* RadDtype of one element */
    uint32_t reserved;
    int64_t  block[2];                    /* weight rows x cols one element covers */
    int64_t  rows, cols;                  /* the element grid */
    int64_t  row_bytes;                   /* pitch of the grid's rows */
    int64_t  offset;                      /* first byte, from the blob's start */
} RadPlanesEntry;

typedef struct RadPlanesHeader {
    uint32_t magic;                       /* RAD_PLANES_MAGIC */
    uint32_t version;                     /* RAD_PLANES_VERSION */
    uint32_t n_planes;
    uint32_t transform[RAD_PLANES_MAX];   /* per plane: 0 = stored as is */
    uint32_t reserved;
    int64_t  bytes;                       /* the whole blob, header included */
    RadPlanesEntry entry[RAD_PLANES_MAX];
} RadPlanesHeader;

/* The header at the start of a blob (host-readable memory), or null without one. */
static inline const RadPlanesHeader* rad_planes_header(const void* blob) {
    const RadPlanesHeader* h = (const RadPlanesHeader*)blob;
    if (!h || h->magic != RAD_PLANES_MAGIC || h->version != RAD_PLANES_VERSION ||
        h->n_planes > RAD_PLANES_MAX)
        return 0;
    return h;
}

/* The plane of role `role` in the blob whose header is `h` (a host copy of it), or null;
 * *e (if given) receives its entry.  The returned address is `base` + the entry's offset,
 * so it points into whichever copy of the blob `base` addresses. */
static inline const void* rad_planes_find_at(const RadPlanesHeader* h, const void* base,
                                            const char* role, const RadPlanesEntry** e) {
    if (!h) return 0;
    for (uint32_t i = 0; i < h->n_planes; ++i)
        if (strncmp(h->entry[i].role, role, RAD_PLANES_ROLE) == 0) {
            if (e) *e = &h->entry[i];
            return (const uint8_t*)base + h->entry[i].offset;
        }
    return 0;
}

static inline const void* rad_planes_find(const void* blob, const char* role,
                                          const RadPlanesEntry** e) {
    return rad_planes_find_at(rad_planes_header(blob), blob, role, e);
}

#ifdef __cplusplus
}
#endif

#endif /* RAD_PLANES_H */
