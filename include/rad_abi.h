/* rad_abi.h -- radiance kernel-plugin ABI, version 26: the subset libr3d's gemm_nt_q
 * rows use, RECONSTRUCTED from how the reference plugin spells it.
 *
 * radiance v1.11.0's own rad_abi.h / rad_types.h are not available offline (the
 * reference image clones them: docker/Dockerfile.dev:16,25-26), so field ORDER follows
 * the reference's positional initialisers and field TYPES its printf formats:
 *   RadTensor     {data, dtype, rank, shape[], stride[]}, strides in ELEMENTS; an FP4
 *                 tensor counts nibbles (tools/probe_m4_entry.cpp:48-55;
 *                 src/r3d_dump.hip:277-282 prints dtype/rank with %u).
 *   RadParam      {kind, key, ival, ihi, sval, dval}  (src/r3d_dump.hip:273-275).
 *   RadArgs       {t, n_t, p, n_p, <2 fields>, scratch, scratch_bytes, <1 field>}
 *                 (tools/bench_gemv_prof.cpp:101, src/r3d_gemm_fp8a8.hip:1218).
 *   RadConstraint {key, op, ival, sval}  (tools/rows_dump.cpp:11-34).
 *   RadKernelInfo {name, op, family, prose x3, domain, priority, constraints,
 *                 n_constraints, tunables, n_tunables, replaces, init, fini, launch,
 *                 scratch, layout, relayout, opd_shape, unrelayout}
 *                 (src/r3d_rows.cpp:1033-1036, 1601-1675).
 *   RadOpSchema   {op, params, n_params, operands, n_operands, prose}
 *                 (src/r3d_rows.cpp:793-850).
 *   RadEncoding   {scheme, n_planes, transform[], plane[]}, RadEncPlane {role, kind,
 *                 dtype, block[2]}, RadLayout {tag, ...} and the three weight-layout hook
 *                 signatures, from the hooks' uses (src/r3d_gemm_logits.hip:233-272,
 *                 src/r3d_gemm_w2a8.hip:1362-1436, src/r3d_rows.cpp:1353-1358): roles and
 *                 the scheme are fixed-size strings compared with strncmp(.., RAD_ENC_STR),
 *                 `transform[0]` non-zero means a rotated encoding, `kind` is
 *                 RAD_PLANE_TILED for a plain element grid, and at declare time the plane
 *                 tensors carry geometry with null data.
 * Enum VALUES and the array bound RAD_MAX_RANK are not recoverable from the reference
 * and are this header's own; the whole dependency is isolated here so the real v1.11.0
 * header can replace this file without touching any other source.
 */
#ifndef RAD_ABI_H
#define RAD_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RAD_ABI_VERSION 26u
#define RAD_MAX_RANK 8

/* Engine stream handle; on ROCm it is a hipStream_t (src/r3d_gemm_mxfp4.hip:1616). */
typedef void* RadStream;

enum RadDtype {
    RAD_F32 = 0, RAD_BF16, RAD_F16, RAD_F8E4M3, RAD_F8E5M2, RAD_FP4E2M1, RAD_E8M0,
    RAD_U8, RAD_I8, RAD_I16, RAD_I32, RAD_U32, RAD_I64, RAD_BOOL,
    RAD_U4, RAD_U2                        /* sub-byte code planes (src/r3d_gemm_w2a8.hip:1382,1388) */
};

/* Return codes: RAD_OK is zero, every refusal non-zero (entries test `if (rc)`). */
enum RadStatus {
    RAD_OK = 0, RAD_E_UNSUPPORTED = 1, RAD_E_SHAPE = 2, RAD_E_STRIDE = 3,
    RAD_E_DTYPE = 4, RAD_E_INVAL = 5, RAD_E_DEVICE = 6
};

typedef struct RadTensor {
    void*    data;
    uint32_t dtype;
    uint32_t rank;
    int64_t  shape[RAD_MAX_RANK];
    int64_t  stride[RAD_MAX_RANK];        /* elements; FP4 counts nibbles */
} RadTensor;

enum RadParamKind { RAD_P_INT = 0, RAD_P_STR = 1, RAD_P_F64 = 2 };

typedef struct RadParam {
    int         kind;
    const char* key;
    long long   ival;
    long long   ihi;
    const char* sval;
    double      dval;
} RadParam;

#define RAD_INT(k, v) { RAD_P_INT, (k), (long long)(v), 0, (const char*)0, 0.0 }
#define RAD_STR(k, s) { RAD_P_STR, (k), 0, 0, (s), 0.0 }
#define RAD_F64(k, d) { RAD_P_F64, (k), 0, 0, (const char*)0, (double)(d) }

typedef struct RadTunableValue {
    const char* name;
    long long   value;
} RadTunableValue;

typedef struct RadArgs {
    const RadTensor*       t;             /* operands in schema order; absent: data == 0 */
    int                    n_t;
    const RadParam*        p;
    int                    n_p;
    const RadTunableValue* tv;            /* per-row tunables chosen by the engine */
    int                    n_tv;
    void*                  scratch;       /* launch scratch sized by the row's hook */
    int64_t                scratch_bytes;
    uint32_t               flags;
} RadArgs;

enum RadConstraintOp { RAD_C_EQ = 0, RAD_C_LE = 1, RAD_C_GE = 2, RAD_C_DIV = 3, RAD_C_IN = 4 };

/* A constraint on a key the query does not carry never holds. */
typedef struct RadConstraint {
    const char* key;
    int         op;
    long long   ival;
    const char* sval;                     /* RAD_C_IN: space-separated accepted strings */
} RadConstraint;

typedef struct RadTunable {
    const char*      name;
    const long long* values;
    int              n_values;
    int              def;
    const char*      prose;
} RadTunable;

enum RadDomain { RAD_DOMAIN_HOST = 0, RAD_DOMAIN_DEVICE = 1 };

/* A weight's encoding as the engine declares it to a row's layout hooks. */
#define RAD_ENC_STR 16
#define RAD_ENC_MAX_PLANES 4

enum RadPlaneKind { RAD_PLANE_TILED = 0 };   /* one element per block[0] x block[1] weights */

typedef struct RadEncPlane {
    char     role[RAD_ENC_STR];           /* "codes", "scale", "zero", ... NUL-padded */
    uint32_t kind;                        /* RadPlaneKind */
    uint32_t dtype;                       /* RadDtype of one element */
    int64_t  block[2];                    /* weight rows x cols one element covers */
} RadEncPlane;

typedef struct RadEncoding {
    char        scheme[RAD_ENC_STR];      /* "affine", ... */
    int         n_planes;
    uint32_t    transform[RAD_ENC_MAX_PLANES];   /* [0] non-zero: a rotated encoding */
    RadEncPlane plane[RAD_ENC_MAX_PLANES];
} RadEncoding;

/* What a layout hook answers: the name of the device layout and the bytes its relayout
 * writes. */
typedef struct RadLayout {
    const char* tag;
    int64_t     bytes;
} RadLayout;

typedef int     (*RadInitFn)(void);
typedef void    (*RadFiniFn)(void);
typedef int     (*RadLaunchFn)(const RadArgs* a, RadStream s);
typedef int64_t (*RadScratchFn)(const RadArgs* a);
/* Weight-layout hooks, host only.  `operand` is the schema index of the weight, `sel[i]`
 * the encoding plane that planes[i] holds.  layout: RAD_OK and *out, RAD_E_UNSUPPORTED for
 * "store the operand as it is", any other code declines the row for this weight.
 * relayout writes the device form into dst (host memory of dst_bytes); unrelayout reads
 * it back into the planes. */
typedef int (*RadLayoutFn)(const RadParam* p, int n_p, int operand, const RadEncoding* enc,
                           const int* sel, const RadTensor* planes, int n, RadLayout* out);
typedef int (*RadRelayoutFn)(const RadParam* p, int n_p, int operand, const RadEncoding* enc,
                             const int* sel, const RadTensor* planes, int n, void* dst,
                             int64_t dst_bytes);
typedef int (*RadUnrelayoutFn)(const RadParam* p, int n_p, int operand,
                               const RadEncoding* enc, const int* sel, const void* src,
                               int64_t src_bytes, const RadTensor* planes, int n);

typedef struct RadKernelInfo {
    const char*          name;
    const char*          op;
    const char*          family;
    const char*          summary;
    const char*          limits;
    const char*          formats;
    int                  domain;
    int                  priority;
    const RadConstraint* constraints;
    int                  n_constraints;
    const RadTunable*    tunables;
    int                  n_tunables;
    const char*          replaces;        /* fused rows only; zero for a plain row */
    RadInitFn            init;
    RadFiniFn            fini;
    RadLaunchFn          launch;
    RadScratchFn         scratch;
    RadLayoutFn          layout;          /* weight layout hooks (null: none) */
    RadRelayoutFn        relayout;
    const void*          opd_shape;       /* unused by these rows */
    RadUnrelayoutFn      unrelayout;
} RadKernelInfo;

enum RadParamReq { RAD_REQUIRED = 0, RAD_OPTIONAL = 1, RAD_DERIVED = 2 };
enum RadOperandRole { RAD_OPD_IN = 0, RAD_OPD_OUT = 1, RAD_OPD_INOUT = 2, RAD_OPD_WEIGHT = 3 };

typedef struct RadParamSpec {
    const char* key;
    int         kind;
    int         req;
    int         role;
} RadParamSpec;

typedef struct RadOperandSpec {
    const char* name;
    int         role;
    int         optional;
} RadOperandSpec;

typedef struct RadOpSchema {
    const char*           op;
    const RadParamSpec*   params;
    int                   n_params;
    const RadOperandSpec* operands;
    int                   n_operands;
    const char*           prose;
} RadOpSchema;

enum RadPluginKind { RAD_PLUGIN_KERNEL = 1 };

typedef struct RadPluginInfo {
    int         kind;
    const char* name;
    const char* version;
    const char* description;
    const char* targets;
} RadPluginInfo;

#ifdef __cplusplus
}
#endif

#endif /* RAD_ABI_H */
