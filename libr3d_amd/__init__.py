"""libr3d_amd -- Python host mirror of the gfx950 gemm_nt_q rows (libr3d_gfx950.so).

The shared library is the product: a radiance kernel plugin (ABI 26) whose rows are
reached through ``rad_kernel_at(i)->launch(const RadArgs*, RadStream)``.  This module
binds that C ABI with ctypes -- the structures below mirror ``include/rad_abi.h`` field
for field -- and adds what an engine would do around it: build ``RadArgs`` from device
tensors and resolve a row per op and band (constraints + priority, the resolver the
reference describes at src/r3d_rows.cpp:1105-1110,1165-1177).

PyTorch is used only for device memory and streams.  Every compute call goes through the
HIP library; if the library is missing this module raises instead of computing anything
another way.
"""
import ctypes
import os

__all__ = [
    "RAD_OK", "RAD_E_UNSUPPORTED", "RAD_E_SHAPE", "RAD_E_STRIDE", "RAD_E_DTYPE",
    "RAD_E_INVAL", "RAD_E_DEVICE", "DT", "RadTensor", "RadParam", "RadArgs",
    "RadKernelInfo", "RadOpSchema", "lib", "lib_path", "rows", "schemas", "resolve",
    "launch_row", "gemm_nt_q", "describe", "GemmOperands", "QuantActOperands", "quant_act_fp8",
    "GatedQuantOperands", "GatedGemmOperands", "RmsNormQuantOperands", "build_id",
    "check_build_id", "mxfp4a16_stage", "LogitsOperands", "logits_gemm", "head_bytes",
    "join_head", "split_head", "forget_head", "head_header", "RadEncoding", "RadEncPlane",
    "RadLayout", "RadPlanesHeader", "RadPlanesEntry", "head_encoding", "layout_head",
    "relayout_head", "unrelayout_head",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
lib_path = os.path.join(_HERE, "libr3d_gfx950.so")

RAD_MAX_RANK = 8
RAD_OK, RAD_E_UNSUPPORTED, RAD_E_SHAPE, RAD_E_STRIDE, RAD_E_DTYPE, RAD_E_INVAL, RAD_E_DEVICE = range(7)

# enum RadDtype (include/rad_abi.h)
DT = {name: i for i, name in enumerate(
    ["F32", "BF16", "F16", "F8E4M3", "F8E5M2", "FP4E2M1", "E8M0", "U8", "I8", "I16", "I32",
     "U32", "I64", "BOOL", "U4", "U2"])}
RAD_P_INT, RAD_P_STR, RAD_P_F64 = 0, 1, 2
RAD_C_EQ, RAD_C_LE, RAD_C_GE, RAD_C_DIV, RAD_C_IN = range(5)


class RadTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_uint32), ("rank", ctypes.c_uint32),
                ("shape", ctypes.c_int64 * RAD_MAX_RANK), ("stride", ctypes.c_int64 * RAD_MAX_RANK)]


class RadParam(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("key", ctypes.c_char_p), ("ival", ctypes.c_longlong),
                ("ihi", ctypes.c_longlong), ("sval", ctypes.c_char_p), ("dval", ctypes.c_double)]


class RadTunableValue(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("value", ctypes.c_longlong)]


class RadTunable(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("values", ctypes.POINTER(ctypes.c_longlong)),
                ("n_values", ctypes.c_int), ("def", ctypes.c_int), ("prose", ctypes.c_char_p)]


class RadArgs(ctypes.Structure):
    _fields_ = [("t", ctypes.POINTER(RadTensor)), ("n_t", ctypes.c_int),
                ("p", ctypes.POINTER(RadParam)), ("n_p", ctypes.c_int),
                ("tv", ctypes.POINTER(RadTunableValue)), ("n_tv", ctypes.c_int),
                ("scratch", ctypes.c_void_p), ("scratch_bytes", ctypes.c_int64),
                ("flags", ctypes.c_uint32)]


class RadConstraint(ctypes.Structure):
    _fields_ = [("key", ctypes.c_char_p), ("op", ctypes.c_int), ("ival", ctypes.c_longlong),
                ("sval", ctypes.c_char_p)]


LaunchFn = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(RadArgs), ctypes.c_void_p)
ScratchFn = ctypes.CFUNCTYPE(ctypes.c_int64, ctypes.POINTER(RadArgs))


class RadKernelInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("op", ctypes.c_char_p), ("family", ctypes.c_char_p),
                ("summary", ctypes.c_char_p), ("limits", ctypes.c_char_p),
                ("formats", ctypes.c_char_p), ("domain", ctypes.c_int),
                ("priority", ctypes.c_int), ("constraints", ctypes.POINTER(RadConstraint)),
                ("n_constraints", ctypes.c_int), ("tunables", ctypes.POINTER(RadTunable)),
                ("n_tunables", ctypes.c_int), ("replaces", ctypes.c_char_p),
                ("init", ctypes.c_void_p), ("fini", ctypes.c_void_p), ("launch", ctypes.c_void_p),
                ("scratch", ctypes.c_void_p), ("layout", ctypes.c_void_p),
                ("relayout", ctypes.c_void_p), ("opd_shape", ctypes.c_void_p),
                ("unrelayout", ctypes.c_void_p)]


RAD_ENC_STR, RAD_ENC_MAX_PLANES, RAD_PLANE_TILED = 16, 4, 0


class RadEncPlane(ctypes.Structure):
    _fields_ = [("role", ctypes.c_char * RAD_ENC_STR), ("kind", ctypes.c_uint32),
                ("dtype", ctypes.c_uint32), ("block", ctypes.c_int64 * 2)]


class RadEncoding(ctypes.Structure):
    _fields_ = [("scheme", ctypes.c_char * RAD_ENC_STR), ("n_planes", ctypes.c_int),
                ("transform", ctypes.c_uint32 * RAD_ENC_MAX_PLANES),
                ("plane", RadEncPlane * RAD_ENC_MAX_PLANES)]


class RadLayout(ctypes.Structure):
    _fields_ = [("tag", ctypes.c_char_p), ("bytes", ctypes.c_int64)]


class RadPlanesHeader(ctypes.Structure):          # include/rad_planes.h
    _fields_ = [("magic", ctypes.c_uint32), ("n_planes", ctypes.c_uint32),
                ("transform", ctypes.c_uint32 * 4), ("bytes", ctypes.c_int64)]


class RadPlanesEntry(ctypes.Structure):
    _fields_ = [("role", ctypes.c_char * 16), ("dtype", ctypes.c_uint32), ("kind", ctypes.c_uint32),
                ("block", ctypes.c_int64 * 2), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                ("row_bytes", ctypes.c_int64), ("offset", ctypes.c_int64)]


class RadParamSpec(ctypes.Structure):
    _fields_ = [("key", ctypes.c_char_p), ("kind", ctypes.c_int), ("req", ctypes.c_int),
                ("role", ctypes.c_int)]


class RadOperandSpec(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("role", ctypes.c_int), ("optional", ctypes.c_int)]


class RadOpSchema(ctypes.Structure):
    _fields_ = [("op", ctypes.c_char_p), ("params", ctypes.POINTER(RadParamSpec)),
                ("n_params", ctypes.c_int), ("operands", ctypes.POINTER(RadOperandSpec)),
                ("n_operands", ctypes.c_int), ("prose", ctypes.c_char_p)]


class RadPluginInfo(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("name", ctypes.c_char_p), ("version", ctypes.c_char_p),
                ("description", ctypes.c_char_p), ("targets", ctypes.c_char_p)]


_LIB = None


def lib():
    """The loaded libr3d_gfx950.so (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(lib_path):
            raise RuntimeError("libr3d_gfx950.so is not built (run __graft_entry__.build() or "
                               "python -m libr3d_amd.build): %s" % lib_path)
        L = ctypes.CDLL(lib_path)
        L.rad_plugin_abi_version.restype = ctypes.c_uint32
        L.rad_plugin_info.restype = ctypes.POINTER(RadPluginInfo)
        L.rad_kernel_schema_count.restype = ctypes.c_int
        L.rad_kernel_schema_at.restype = ctypes.POINTER(RadOpSchema)
        L.rad_kernel_schema_at.argtypes = [ctypes.c_int]
        L.rad_kernel_count.restype = ctypes.c_int
        L.rad_kernel_at.restype = ctypes.POINTER(RadKernelInfo)
        L.rad_kernel_at.argtypes = [ctypes.c_int]
        for name in ("r3d_rad_gemm_nt_q", "r3d_rad_gemm_nt_q_mxfp4_decode",
                     "r3d_rad_gemm_nt_q_fp8", "r3d_rad_gemm_nt_q_fp8_decode"):
            fn = getattr(L, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.POINTER(RadArgs), ctypes.c_void_p]
        L.r3d_gfx950_describe.restype = ctypes.c_int
        L.r3d_gfx950_describe.argtypes = [ctypes.c_char_p, ctypes.POINTER(RadArgs),
                                          ctypes.c_char_p, ctypes.c_int]
        L.r3d_gfx950_mxfp4a16_stage.restype = ctypes.c_int
        L.r3d_gfx950_mxfp4a16_stage.argtypes = [ctypes.POINTER(RadArgs), ctypes.c_void_p,
                                                ctypes.c_int]
        L.r3d_gfx950_build_id.restype = ctypes.c_char_p
        L.r3d_gfx950_build_id.argtypes = []
        _i64 = ctypes.c_int64
        L.r3d_gfx950_logits_head_bytes.restype = _i64
        L.r3d_gfx950_logits_head_bytes.argtypes = [_i64, _i64, ctypes.c_uint32, _i64]
        L.r3d_gfx950_logits_head_header.restype = _i64
        L.r3d_gfx950_logits_head_header.argtypes = [_i64, _i64, ctypes.c_uint32, _i64,
                                                    ctypes.c_void_p]
        L.r3d_gfx950_logits_head_join.restype = ctypes.c_int
        L.r3d_gfx950_logits_head_join.argtypes = [
            ctypes.c_void_p, _i64, ctypes.c_void_p, _i64, _i64, _i64, ctypes.c_uint32, _i64,
            ctypes.c_void_p, _i64]
        L.r3d_gfx950_logits_head_split.restype = ctypes.c_int
        L.r3d_gfx950_logits_head_split.argtypes = [ctypes.c_void_p, _i64, ctypes.c_void_p,
                                                   ctypes.c_void_p]
        _hook = [ctypes.POINTER(RadParam), ctypes.c_int, ctypes.c_int, ctypes.POINTER(RadEncoding),
                 ctypes.POINTER(ctypes.c_int), ctypes.POINTER(RadTensor), ctypes.c_int]
        L.r3d_layout_head.restype = ctypes.c_int
        L.r3d_layout_head.argtypes = _hook + [ctypes.POINTER(RadLayout)]
        L.r3d_relayout_head.restype = ctypes.c_int
        L.r3d_relayout_head.argtypes = _hook + [ctypes.c_void_p, _i64]
        L.r3d_unrelayout_head.restype = ctypes.c_int
        L.r3d_unrelayout_head.argtypes = _hook[:5] + [ctypes.c_void_p, _i64,
                                                       ctypes.POINTER(RadTensor), ctypes.c_int]
        L.r3d_gfx950_stream_probe.restype = ctypes.c_int
        L.r3d_gfx950_stream_probe.argtypes = [ctypes.c_void_p, _i64, ctypes.c_int, _i64,
                                              ctypes.c_void_p, ctypes.c_void_p]
        L.r3d_gfx950_mfma_valu_probe.restype = ctypes.c_int
        L.r3d_gfx950_mfma_valu_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.r3d_gfx950_logits_head_forget.restype = None
        L.r3d_gfx950_logits_head_forget.argtypes = [ctypes.c_void_p]
        _LIB = L
    return _LIB


def _s(b):
    return b.decode() if isinstance(b, bytes) else b


def build_id():
    """The SHA-256 of the sources the loaded library was compiled from."""
    return _s(lib().r3d_gfx950_build_id())


def check_build_id():
    """Raise unless the loaded library was built from the sources beside this module (a
    stale binary would test or benchmark other code than the tree holds)."""
    from libr3d_amd import build as B
    got, want = build_id(), B.source_id()
    if got != want:
        raise RuntimeError("libr3d_gfx950.so is stale: built from sources %s, tree holds %s "
                           "(rebuild: python -m libr3d_amd.build)" % (got[:16], want[:16]))
    return got


def mxfp4a16_stage(ops, stage, stream=0):
    """One stage of a gemm_nt_q_mxfp4a16 call (0 whole, 1 quantiser, 2 GEMM on the planes
    already in the scratch); returns the status."""
    return lib().r3d_gfx950_mxfp4a16_stage(ctypes.byref(ops.args), ctypes.c_void_p(stream),
                                           int(stage))


def rows():
    """The registered rows as dicts (after the registration-time kill switches)."""
    L = lib()
    out = []
    for i in range(L.rad_kernel_count()):
        k = L.rad_kernel_at(i).contents
        cons = [(_s(k.constraints[c].key), k.constraints[c].op, k.constraints[c].ival,
                 _s(k.constraints[c].sval)) for c in range(k.n_constraints)]
        tun = [_s(k.tunables[t].name) for t in range(k.n_tunables)]
        out.append({"name": _s(k.name), "op": _s(k.op), "priority": k.priority,
                    "domain": k.domain, "constraints": cons, "tunables": tun, "launch": k.launch,
                    "scratch": k.scratch, "layout": k.layout, "relayout": k.relayout,
                    "opd_shape": k.opd_shape, "unrelayout": k.unrelayout})
    return out


def schemas():
    L = lib()
    out = []
    for i in range(L.rad_kernel_schema_count()):
        s = L.rad_kernel_schema_at(i).contents
        out.append({
            "op": _s(s.op),
            "params": [(_s(s.params[j].key), s.params[j].kind, s.params[j].req)
                       for j in range(s.n_params)],
            "operands": [(_s(s.operands[j].name), s.operands[j].role, s.operands[j].optional)
                         for j in range(s.n_operands)],
        })
    return out


def _holds(c, query):
    key, op, ival, sval = c
    if key not in query:
        return False                     # a constraint on an absent key never holds
    v = query[key]
    if op == RAD_C_IN:
        return isinstance(v, str) and v in (sval or "").split()
    if isinstance(v, str):
        return False
    if op == RAD_C_EQ:
        return v == ival
    if op == RAD_C_LE:
        return v <= ival
    if op == RAD_C_GE:
        return v >= ival
    if op == RAD_C_DIV:
        return ival != 0 and v % ival == 0
    return False


def resolve(op, query):
    """Highest-priority registered row of `op` whose constraints all hold, or None."""
    best = None
    for r in rows():
        if r["op"] != op:
            continue
        if all(_holds(c, query) for c in r["constraints"]):
            if best is None or r["priority"] > best["priority"]:
                best = r
    return best


class GemmOperands:
    """Owns the ctypes RadArgs for one gemm_nt_q call over device tensors.

    a      uint8 [M, K]           e4m3 codes (mxfp4a16: bf16/int16 [M, K])
    a_scale float32 [M, K/128]    (mxfp4a16: None)
           The decode rows also take a bf16/int16 `a` with a_scale None: the GEMV quantises
           it with quant_act_fp8's arithmetic (groups of 128) on the way into its LDS.
    b      uint8 [N, K/2] (mxfp4a8/a16: packed e2m1, low nibble = even k) or [N, K] (fp8a8)
    b_scale uint8 [N, K/32] E8M0 (mxfp4) or bf16/int16 [N or N/128, K/128] (fp8a8)
    y      bf16/int16 [M, N]
    scratch optional device tensor handed over as RadArgs::scratch (mxfp4a16)
    """

    def __init__(self, a, a_scale, b, b_scale, y, *, dtype, N, K, group=None, M=None,
                 a_sum=None, b_ref=None, extra_params=None, y_shape=None, tunables=None,
                 scratch=None):
        mx = dtype in ("mxfp4a8", "mxfp4a16")
        self.dtype = dtype
        group = group if group is not None else (32 if mx else 128)
        t = (RadTensor * 7)()

        def fill(i, x, dt, shape=None, stride=None):
            if x is None:
                t[i].data = None
                t[i].rank = 0
                return
            t[i].data = x.data_ptr()
            t[i].dtype = DT[dt]
            shp = list(shape if shape is not None else x.shape)
            std = list(stride if stride is not None else x.stride())
            t[i].rank = len(shp)
            for r, (s_, st) in enumerate(zip(shp, std)):
                t[i].shape[r] = int(s_)
                t[i].stride[r] = int(st)

        # the launch reads raw pointers: hold the tensors so none is freed (and its memory
        # reused) while this object can still launch
        self._tensors = [a, a_scale, b, b_scale, y, a_sum, b_ref]
        fused = a is not None and a_scale is None and a.element_size() == 2
        fill(0, a, "BF16" if dtype == "mxfp4a16" or fused else "F8E4M3")
        fill(1, a_scale, "F32")
        if mx:
            # FP4 counts nibbles: [N, K] with strides {K, 1}
            fill(2, b, "FP4E2M1", [b.shape[0], b.shape[1] * 2], [b.stride(0) * 2, 1])
            fill(3, b_scale, "E8M0")
        else:
            fill(2, b, "F8E4M3")
            fill(3, b_scale, "BF16")
        fill(4, y, "BF16", y_shape)
        fill(5, a_sum, "F32")
        fill(6, b_ref, "BF16")
        self._t = t
        params = [("dtype", dtype), ("N", int(N)), ("K", int(K)), ("group", int(group))]
        if M is not None:
            params.append(("M", int(M)))
        params += list(extra_params or [])
        p = (RadParam * len(params))()
        self._keep = []
        for i, (k, v) in enumerate(params):
            kb = k.encode()
            self._keep.append(kb)
            p[i].key = kb
            if isinstance(v, str):
                vb = v.encode()
                self._keep.append(vb)
                p[i].kind = RAD_P_STR
                p[i].sval = vb
            elif isinstance(v, float):
                p[i].kind = RAD_P_F64
                p[i].dval = v
            else:
                p[i].kind = RAD_P_INT
                p[i].ival = v
        self._p = p
        tunables = list(tunables or [])
        tv = (RadTunableValue * max(1, len(tunables)))()
        for i, (k, v) in enumerate(tunables):
            kb = k.encode()
            self._keep.append(kb)
            tv[i].name = kb
            tv[i].value = int(v)
        self._tv = tv
        self.args = RadArgs(ctypes.cast(t, ctypes.POINTER(RadTensor)), 7,
                            ctypes.cast(p, ctypes.POINTER(RadParam)), len(params),
                            ctypes.cast(tv, ctypes.POINTER(RadTunableValue)), len(tunables),
                            None, 0, 0)
        if scratch is not None:
            self.set_scratch(scratch)

    def set_scratch(self, scratch, nbytes=None):
        """Hand `scratch` (a device tensor) to the launch as RadArgs::scratch."""
        self._scratch = scratch
        self.args.scratch = scratch.data_ptr()
        self.args.scratch_bytes = int(nbytes if nbytes is not None
                                      else scratch.numel() * scratch.element_size())

    def set_y(self, y):
        self._tensors[4] = y
        self._t[4].data = y.data_ptr()


class QuantActOperands:
    """Owns the ctypes RadArgs for one quant_act_fp8 call (src/r3d_band.hip:460-487).

    x     float32 or bf16/int16 [M, n] (any view the band walk accepts; rank 1 is one row)
    q     uint8 [M, n]                    e4m3 codes out
    scale float32 [M, ceil(n / group)]    dequant scales out
    x_dtype "F32" or "BF16" names x's element type (int16 tensors carry bf16 bits).
    """

    def __init__(self, x, q, scale, *, n, group, M=None, x_dtype=None, dtype=None,
                 shapes=None, strides=None):
        t = (RadTensor * 3)()
        self._tensors = [x, q, scale]                 # held while this object can launch
        xdt = x_dtype or ("F32" if str(x.dtype).endswith("float32") else "BF16")
        shapes = shapes or {}
        strides = strides or {}
        for i, (ten, dt) in enumerate(((x, xdt), (q, "F8E4M3"), (scale, "F32"))):
            if ten is None:
                t[i].data = None
                t[i].rank = 0
                continue
            t[i].data = ten.data_ptr()
            t[i].dtype = DT[dt]
            shp = list(shapes.get(i, ten.shape))
            std = list(strides.get(i, ten.stride()))
            t[i].rank = len(shp)
            for r, (s_, st) in enumerate(zip(shp, std)):
                t[i].shape[r] = int(s_)
                t[i].stride[r] = int(st)
        self._t = t
        params = [("n", int(n)), ("group", int(group)),
                  ("dtype", dtype or ("f32" if xdt == "F32" else "bf16"))]
        if M is not None:
            params.append(("M", int(M)))
        p = (RadParam * len(params))()
        self._keep = []
        for i, (k, v) in enumerate(params):
            kb = k.encode()
            self._keep.append(kb)
            p[i].key = kb
            if isinstance(v, str):
                vb = v.encode()
                self._keep.append(vb)
                p[i].kind = RAD_P_STR
                p[i].sval = vb
            else:
                p[i].kind = RAD_P_INT
                p[i].ival = v
        self._p = p
        self.args = RadArgs(ctypes.cast(t, ctypes.POINTER(RadTensor)), 3,
                            ctypes.cast(p, ctypes.POINTER(RadParam)), len(params),
                            None, 0, None, 0, 0)


class _Args:
    """ctypes RadArgs over operands [(tensor or None, element type name, shape, stride)]
    (shape / stride None: the tensor's own) and params [(key, int | float | str)]."""

    def __init__(self, operands, params):
        t = (RadTensor * len(operands))()
        self._tensors = [op[0] for op in operands]   # held while this object can launch
        for i, (ten, dt, shp, std) in enumerate(operands):
            if ten is None:
                t[i].data = None
                t[i].rank = 0
                continue
            t[i].data = ten.data_ptr()
            t[i].dtype = DT[dt]
            shp = list(shp if shp is not None else ten.shape)
            std = list(std if std is not None else ten.stride())
            t[i].rank = len(shp)
            for r, (s_, st) in enumerate(zip(shp, std)):
                t[i].shape[r] = int(s_)
                t[i].stride[r] = int(st)
        self._t = t
        p = (RadParam * max(1, len(params)))()
        self._keep = []
        for i, (k, v) in enumerate(params):
            kb = k.encode()
            self._keep.append(kb)
            p[i].key = kb
            if isinstance(v, str):
                vb = v.encode()
                self._keep.append(vb)
                p[i].kind = RAD_P_STR
                p[i].sval = vb
            elif isinstance(v, float):
                p[i].kind = RAD_P_F64
                p[i].dval = v
            else:
                p[i].kind = RAD_P_INT
                p[i].ival = int(v)
        self._p = p
        self.args = RadArgs(ctypes.cast(t, ctypes.POINTER(RadTensor)), len(operands),
                            ctypes.cast(p, ctypes.POINTER(RadParam)), len(params),
                            None, 0, None, 0, 0)

    def set_scratch(self, scratch, nbytes=None):
        """Hand `scratch` (a device tensor) to the launch as RadArgs::scratch."""
        self._scratch = scratch
        self.args.scratch = scratch.data_ptr()
        self.args.scratch_bytes = int(nbytes if nbytes is not None
                                      else scratch.numel() * scratch.element_size())


def _elt(x, default="BF16"):
    return "F32" if str(x.dtype).endswith("float32") else default


class GatedQuantOperands(_Args):
    """One gated_quant_fp8 call (src/r3d_band.hip:492-541).

    gate_up float32 or bf16/int16 [M, 2n]   gate columns [0, n), up columns [n, 2n)
    q       uint8 [M, n]                      e4m3 codes out
    scale   float32 [M, ceil(n / group)]      dequant scales out
    out     optional float32 or bf16/int16 [M, n]: the gated value h
    act     "silu" (default when absent) or "sigmoid"
    """

    def __init__(self, gate_up, q, scale, out=None, *, n, group=128, act=None, M=None,
                 dtype=None, shapes=None, strides=None):
        shapes, strides = shapes or {}, strides or {}
        gdt = _elt(gate_up)
        ops = [(gate_up, gdt), (q, "F8E4M3"), (scale, "F32"),
               (out, _elt(out) if out is not None else "BF16")]
        super().__init__([(x, dt, shapes.get(i), strides.get(i)) for i, (x, dt) in enumerate(ops)],
                         [("n", n), ("group", group),
                          ("dtype", dtype or ("f32" if gdt == "F32" else "bf16"))] +
                         ([("act", act)] if act is not None else []) +
                         ([("M", M)] if M is not None else []))


class RmsNormQuantOperands(_Args):
    """One rmsnorm_quant_fp8 call (src/r3d_more.hip:482-539).

    x        bf16/int16 [M, n]
    residual optional bf16/int16 [M, n], updated in place with bf16(residual + x)
    w        float32 or bf16/int16 [n] (rank 1)
    q        uint8 [M, n] e4m3 codes out; scale float32 [M, ceil(n / group)] out
    out      optional float32 or bf16/int16 [M, n]: the normed bf16 values
    """

    def __init__(self, x, residual, w, q, scale, out=None, *, n, eps=1e-6, group=128,
                 wadd=None, M=None, w_dtype=None):
        ops = [(x, "BF16"), (residual, "BF16"), (w, w_dtype or _elt(w)), (q, "F8E4M3"),
               (scale, "F32"), (out, _elt(out) if out is not None else "BF16")]
        super().__init__([(t, dt, None, None) for t, dt in ops],
                         [("n", n), ("eps", float(eps)), ("group", group), ("dtype", "bf16")] +
                         ([("wadd", float(wadd))] if wadd is not None else []) +
                         ([("M", M)] if M is not None else []))


class GatedGemmOperands(_Args):
    """One gemm_nt_q_gated call at fp8a8 (src/r3d_gemm_fp8a8.hip:1166-1241).

    a uint8 [M, K] e4m3, a_scale float32 [M, K/128], b uint8 [N, K] e4m3 (N = 2n: gate rows
    then up rows), b_scale bf16/int16 [N or N/128, K/128], q uint8 [M, n], scale float32
    [M, n/group], out optional float32 or bf16/int16 [M, n]; the launch scratch (the row's
    hook sizes it) holds the [M, N] bf16 gate_up plane.
    """

    def __init__(self, a, a_scale, b, b_scale, q, scale, out=None, *, N, K, act="silu",
                 group=128, M=None, a_sum=None, scratch=None):
        ops = [(a, "F8E4M3"), (a_scale, "F32"), (b, "F8E4M3"), (b_scale, "BF16"),
               (q, "F8E4M3"), (scale, "F32"),
               (out, _elt(out) if out is not None else "BF16")]
        if a_sum is not None:
            ops.append((a_sum, "F32"))
        super().__init__([(x, dt, None, None) for x, dt in ops],
                         [("N", N), ("K", K), ("group", group), ("dtype", "fp8a8")] +
                         ([("act", act)] if act is not None else []) +
                         ([("M", M)] if M is not None else []))
        if scratch is not None:
            self.set_scratch(scratch)


class LogitsOperands(_Args):
    """One logits_gemm call (src/r3d_gemm_logits.hip:144-226).

    x        bf16/int16 [M, n_embd]
    lm_head  uint8 [bytes]: a joined head (join_head) in device memory
    logits   float32 [M, n_vocab] out
    """

    def __init__(self, x, lm_head, logits, *, n_vocab, n_embd, M=None, dtype="bf16",
                 shapes=None, strides=None):
        shapes, strides = shapes or {}, strides or {}
        ops = [(x, "BF16"), (lm_head, "U8"), (logits, "F32")]
        super().__init__([(t, dt, shapes.get(i), strides.get(i)) for i, (t, dt) in enumerate(ops)],
                         [("M", M if M is not None else logits.numel() // n_vocab),
                          ("n_vocab", n_vocab), ("n_embd", n_embd), ("dtype", dtype)])


_SCALE_DT = {"bf16": "BF16", "f16": "F16", "f32": "F32"}


def head_bytes(n_vocab, n_embd, scale_dtype="bf16", scale_block_rows=1):
    """Bytes of a joined head (negative: the RAD_E_* refusal)."""
    return int(lib().r3d_gfx950_logits_head_bytes(n_vocab, n_embd, DT[_SCALE_DT[scale_dtype]],
                                                  scale_block_rows))


HEAD_BYTES = 320                  # sizeof(RadPlanesHead): the header, then 4 entries
HEADER_BYTES = 32 + 2 * 72        # a two-plane blob's header and its two entries


def head_header(n_vocab, n_embd, scale_dtype="bf16", scale_block_rows=1):
    """(header and entries uint8 [HEADER_BYTES], codes offset, scale offset, blob bytes) of
    a joined head, so its planes can be written straight into device memory at those
    offsets."""
    import numpy as np
    h = np.zeros(HEAD_BYTES, np.uint8)
    nb = int(lib().r3d_gfx950_logits_head_header(n_vocab, n_embd, DT[_SCALE_DT[scale_dtype]],
                                                 scale_block_rows, h.ctypes.data))
    if nb < 0:
        raise ValueError("head refused (%d)" % nb)
    e = h[32:].view(np.int64)          # entries from byte 32: 9 int64 each, offset last
    return h[:HEADER_BYTES].copy(), int(e[8]), int(e[17]), nb


def join_head(codes, scale, scale_dtype="bf16", scale_block_rows=1):
    """The joined-planes blob (numpy uint8, host) of e4m3 codes [n_vocab, n_embd] and a
    scale grid [ceil(n_vocab / scale_block_rows), ceil(n_embd / 128)] (uint16 bits for
    bf16 / f16, float32 for f32), through the library's r3d_gfx950_logits_head_join."""
    import numpy as np
    codes = np.ascontiguousarray(codes, np.uint8)
    scale = np.ascontiguousarray(scale, np.float32 if scale_dtype == "f32" else np.uint16)
    n_vocab, n_embd = codes.shape
    nb = head_bytes(n_vocab, n_embd, scale_dtype, scale_block_rows)
    if nb < 0:
        raise ValueError("head refused (%d)" % nb)
    blob = np.empty(nb, np.uint8)
    rc = lib().r3d_gfx950_logits_head_join(
        codes.ctypes.data, n_embd, scale.ctypes.data, scale.shape[1] * scale.itemsize, n_vocab,
        n_embd, DT[_SCALE_DT[scale_dtype]], scale_block_rows, blob.ctypes.data, nb)
    if rc != RAD_OK:
        raise ValueError("join refused (%d)" % rc)
    return blob


def split_head(blob, n_vocab, n_embd, scale_dtype="bf16", scale_block_rows=1):
    """The dense planes back out of a host blob: (codes [n_vocab, n_embd], scale grid)."""
    import numpy as np
    blob = np.ascontiguousarray(blob, np.uint8)
    codes = np.empty((n_vocab, n_embd), np.uint8)
    sdt = np.float32 if scale_dtype == "f32" else np.uint16
    scale = np.empty(((n_vocab + scale_block_rows - 1) // scale_block_rows, (n_embd + 127) // 128),
                     sdt)
    rc = lib().r3d_gfx950_logits_head_split(blob.ctypes.data, blob.size, codes.ctypes.data,
                                            scale.ctypes.data)
    if rc != RAD_OK:
        raise ValueError("split refused (%d)" % rc)
    return codes, scale


def head_encoding(scale_dtype="bf16", scale_block_rows=1, scheme="affine", roles=("codes", "scale"),
                  code_dtype="F8E4M3", code_block=(1, 1), kinds=(RAD_PLANE_TILED, RAD_PLANE_TILED),
                  transform0=0, n_planes=2):
    """A RadEncoding of a joined lm_head as an engine would declare it (every field
    overridable, so tests can hand the hooks what they must decline)."""
    enc = RadEncoding()
    enc.scheme = scheme.encode()
    enc.n_planes = n_planes
    enc.transform[0] = transform0
    sdt = DT[_SCALE_DT.get(scale_dtype, scale_dtype)]
    for i, (role, kind, dt, blk) in enumerate([
            (roles[0], kinds[0], DT[code_dtype], code_block),
            (roles[1], kinds[1], sdt, (scale_block_rows, 128))]):
        enc.plane[i].role = role.encode()
        enc.plane[i].kind = kind
        enc.plane[i].dtype = dt
        enc.plane[i].block[0], enc.plane[i].block[1] = blk
    return enc


def _head_hook_args(enc, codes, scale, sel, params):
    """ctypes arguments shared by the three hooks: params, encoding, selection and the two
    plane tensors (numpy arrays, (array, dtype name) pairs, or (shape, dtype name) pairs for
    geometry only, as at declare time)."""
    import numpy as np
    ps = (RadParam * max(1, len(params)))()
    keep = []
    for i, (k, v) in enumerate(params):
        kb = k.encode()
        keep.append(kb)
        ps[i].kind, ps[i].key, ps[i].ival = RAD_P_INT, kb, int(v)
    ts = (RadTensor * 2)()
    for i, (arr, dt) in enumerate([(codes, "F8E4M3"), (scale, None)]):
        if isinstance(arr, tuple) and isinstance(arr[0], np.ndarray):
            arr, dt = arr                      # (array, dtype name)
        if isinstance(arr, tuple):
            shape, dname = arr
            data = None
        else:
            shape, data = arr.shape, arr.ctypes.data
            dname = dt or {np.dtype(np.float32): "F32", np.dtype(np.uint16): "BF16"}[arr.dtype]
        ts[i].data = data
        ts[i].dtype = DT[dname]
        ts[i].rank = len(shape)
        for j, n in enumerate(shape):
            ts[i].shape[j] = n
        ts[i].stride[len(shape) - 1] = 1
        if len(shape) == 2:
            ts[i].stride[0] = shape[1]
    sl = (ctypes.c_int * 2)(*sel)
    return ps, len(params), enc, sl, ts, keep


def layout_head(enc, codes, scale, operand=1, sel=(0, 1), params=(), n=2):
    """r3d_layout_head: (status, tag, bytes)."""
    ps, n_p, enc, sl, ts, keep = _head_hook_args(enc, codes, scale, sel, params)
    out = RadLayout()
    rc = lib().r3d_layout_head(ps, n_p, operand, ctypes.byref(enc), sl, ts, n, ctypes.byref(out))
    return rc, (_s(out.tag) if out.tag else None), int(out.bytes)


def relayout_head(enc, codes, scale, dst, operand=1, sel=(0, 1), params=()):
    """r3d_relayout_head into the numpy uint8 buffer dst: the status."""
    ps, n_p, enc, sl, ts, keep = _head_hook_args(enc, codes, scale, sel, params)
    return lib().r3d_relayout_head(ps, n_p, operand, ctypes.byref(enc), sl, ts, 2,
                                   dst.ctypes.data, dst.size)


def unrelayout_head(enc, src, codes, scale, operand=1, sel=(0, 1), params=()):
    """r3d_unrelayout_head from the numpy uint8 blob src into codes / scale: the status."""
    ps, n_p, enc, sl, ts, keep = _head_hook_args(enc, codes, scale, sel, params)
    return lib().r3d_unrelayout_head(ps, n_p, operand, ctypes.byref(enc), sl, src.ctypes.data,
                                     src.size, ts, 2)


def forget_head(lm_head):
    """Drop the library's cached header for the blob at lm_head (tensor or address)."""
    ptr = lm_head if isinstance(lm_head, int) else lm_head.data_ptr()
    lib().r3d_gfx950_logits_head_forget(ctypes.c_void_p(ptr))


def logits_gemm(x, lm_head, logits, *, n_vocab, n_embd, stream=None):
    """Launch the logits_gemm_e4m3 row on `stream` (default the current torch stream)."""
    import torch
    ops = LogitsOperands(x, lm_head, logits, n_vocab=n_vocab, n_embd=n_embd)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    return launch_row("logits_gemm_e4m3", ops, stream)


def quant_act_fp8(x, q, scale, *, n, group=128, stream=None):
    """Launch the quant_act_fp8 row on `stream` (a raw hipStream_t int, default the current
    torch stream).  Returns the row's status."""
    import torch
    ops = QuantActOperands(x, q, scale, n=n, group=group, M=x.numel() // n)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    return launch_row("quant_act_fp8_act", ops, stream)


def row_launcher(row_name):
    """The named row's launch pointer as a callable f(ops, stream) -> status."""
    for r in rows():
        if r["name"] == row_name:
            fn = LaunchFn(r["launch"])

            def call(ops, stream=0):
                return fn(ctypes.byref(ops.args), ctypes.c_void_p(stream))
            return call
    raise KeyError("row %s is not registered" % row_name)


def row_scratch_bytes(row_name, ops):
    """The named row's scratch hook on `ops` (bytes; 0 when the row has no hook)."""
    for r in rows():
        if r["name"] == row_name:
            if not r.get("scratch"):
                return 0
            return int(ScratchFn(r["scratch"])(ctypes.byref(ops.args)))
    raise KeyError("row %s is not registered" % row_name)


def launch_row(row_name, ops, stream=0):
    """Call the named row's launch pointer (as the engine does) and return its status."""
    return row_launcher(row_name)(ops, stream)


def describe(row_name, ops):
    buf = ctypes.create_string_buffer(512)
    rc = lib().r3d_gfx950_describe(row_name.encode(), ctypes.byref(ops.args), buf, 512)
    return rc, buf.value.decode()


def gemm_nt_q(a, a_scale, b, b_scale, y, *, dtype, N, K, group=None, stream=None, row=None):
    """Resolve and launch gemm_nt_q on `stream` (a raw hipStream_t int, default the
    current torch stream), with launch scratch of the size the row's hook asks for.
    Returns (status, row name)."""
    import torch
    ops = GemmOperands(a, a_scale, b, b_scale, y, dtype=dtype, N=N, K=K, group=group)
    M = y.numel() // N
    if row is None:
        r = resolve("gemm_nt_q", {"dtype": dtype, "M": M, "N": N, "K": K,
                                  "group": group if group is not None else (32 if dtype == "mxfp4a8" else 128)})
        if r is None:
            return RAD_E_UNSUPPORTED, None
        row = r["name"]
    need = row_scratch_bytes(row, ops)
    if need > 0:                        # the row's hook sized it, as an engine's arena would
        ops.set_scratch(torch.empty(need, dtype=torch.uint8, device=y.device), need)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    return launch_row(row, ops, stream), row
