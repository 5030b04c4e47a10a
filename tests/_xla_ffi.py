"""A fake XLA runtime for the FFI handlers: ctypes structures with the XLA FFI C ABI layout
(API 0.1) and helpers that build call frames from numpy/torch buffers, the way XLA calls an
exported handler. Used by the CPU handler tests (decode and validation paths) and by the GPU
test that runs the handlers on device buffers."""

import ctypes

c_size = ctypes.c_size_t
c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_vp = ctypes.c_void_p

F16, F32, F64, BF16, U8, S32, S64 = 10, 11, 12, 16, 6, 4, 5
EXECUTE, METADATA = 3, 1


class ExtensionBase(ctypes.Structure):
    pass


ExtensionBase._fields_ = [("struct_size", c_size), ("type", c_i32),
                          ("next", ctypes.POINTER(ExtensionBase))]


class ErrorCreateArgs(ctypes.Structure):
    _fields_ = [("struct_size", c_size), ("extension_start", c_vp), ("message", ctypes.c_char_p),
                ("errc", c_i32)]


class StreamGetArgs(ctypes.Structure):
    _fields_ = [("struct_size", c_size), ("extension_start", c_vp), ("ctx", c_vp),
                ("stream", c_vp)]


ERROR_CREATE = ctypes.CFUNCTYPE(c_vp, ctypes.POINTER(ErrorCreateArgs))
STREAM_GET = ctypes.CFUNCTYPE(c_vp, ctypes.POINTER(StreamGetArgs))


class ApiVersion(ctypes.Structure):
    _fields_ = [("struct_size", c_size), ("extension_start", c_vp), ("major_version", ctypes.c_int),
                ("minor_version", ctypes.c_int)]


class Api(ctypes.Structure):
    _fields_ = [("struct_size", c_size), ("extension_start", c_vp), ("api_version", ApiVersion),
                ("internal_api", c_vp), ("error_create", ERROR_CREATE), ("error_get_message", c_vp),
                ("error_destroy", c_vp), ("handler_register", c_vp), ("stream_get", STREAM_GET)]


class Buffer(ctypes.Structure):
    _fields_ = [("struct_size", c_size), ("extension_start", c_vp), ("dtype", c_i32),
                ("data", c_vp), ("rank", c_i64), ("dims", ctypes.POINTER(c_i64))]


class Args(ctypes.Structure):
    _fields_ = [("struct_size", c_size), ("extension_start", c_vp), ("size", c_i64),
                ("types", ctypes.POINTER(c_i32)), ("args", ctypes.POINTER(c_vp))]


class ByteSpan(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_char_p), ("len", c_size)]


class Scalar(ctypes.Structure):
    _fields_ = [("dtype", c_i32), ("value", c_vp)]


class Attrs(ctypes.Structure):
    _fields_ = [("struct_size", c_size), ("extension_start", c_vp), ("size", c_i64),
                ("types", ctypes.POINTER(c_i32)), ("names", ctypes.POINTER(ctypes.POINTER(ByteSpan))),
                ("attrs", ctypes.POINTER(c_vp))]


class CallFrame(ctypes.Structure):
    _fields_ = [("struct_size", c_size), ("extension_start", ctypes.POINTER(ExtensionBase)),
                ("api", ctypes.POINTER(Api)), ("ctx", c_vp), ("stage", c_i32), ("args", Args),
                ("rets", Args), ("attrs", Attrs), ("future", c_vp)]


class Metadata(ctypes.Structure):
    _fields_ = [("struct_size", c_size), ("api_version", ApiVersion), ("traits", ctypes.c_uint32)]


class MetadataExtension(ctypes.Structure):
    _fields_ = [("extension_base", ExtensionBase), ("metadata", ctypes.POINTER(Metadata))]


class FakeXla:
    """Owns an Api table whose Error_Create records (code, message) and whose Stream_Get returns
    a fixed stream handle; builds call frames and keeps every ctypes object alive."""

    def __init__(self, stream=0, stream_error=False):
        self.errors = []
        self.stream = stream
        self.stream_gets = 0
        self._keep = []

        def error_create(args):
            a = args.contents
            self.errors.append((a.errc, a.message.decode()))
            return len(self.errors)  # any non-null pointer

        def stream_get(args):
            self.stream_gets += 1
            if stream_error:  # XLA's failure: a non-null error pointer, no stream
                return 0xE5
            args.contents.stream = self.stream
            return None

        self._ec = ERROR_CREATE(error_create)
        self._sg = STREAM_GET(stream_get)
        self.api = Api(struct_size=ctypes.sizeof(Api), error_create=self._ec,
                       stream_get=self._sg)

    def buffer(self, dtype, shape, data=0):
        dims = (c_i64 * max(1, len(shape)))(*shape)
        b = Buffer(ctypes.sizeof(Buffer), None, dtype, data, len(shape), dims)
        self._keep += [dims, b]
        return b

    def frame(self, args, rets, attrs=(), stage=EXECUTE, extension=None):
        """args/rets: lists of Buffer; attrs: list of (name, dtype, python value)."""
        def table(bufs):
            types = (c_i32 * max(1, len(bufs)))(*([1] * len(bufs)))
            ptrs = (c_vp * max(1, len(bufs)))(*[ctypes.addressof(b) for b in bufs])
            self._keep += [types, ptrs]
            return Args(ctypes.sizeof(Args), None, len(bufs), types, ptrs)

        names, vals, types = [], [], []
        for name, dt, value in attrs:
            raw = name.encode()
            span = ByteSpan(raw, len(raw))
            store = {F32: ctypes.c_float, F64: ctypes.c_double, S32: ctypes.c_int32,
                     S64: ctypes.c_int64}[dt](value)
            sc = Scalar(dt, ctypes.addressof(store))
            self._keep += [raw, span, store, sc]
            names.append(ctypes.pointer(span))
            vals.append(ctypes.addressof(sc))
            types.append(3)
        n = len(attrs)
        name_arr = (ctypes.POINTER(ByteSpan) * max(1, n))(*names)
        val_arr = (c_vp * max(1, n))(*vals)
        type_arr = (c_i32 * max(1, n))(*types)
        self._keep += [name_arr, val_arr, type_arr]
        at = Attrs(ctypes.sizeof(Attrs), None, n, type_arr, name_arr, val_arr)
        ext = ctypes.cast(ctypes.pointer(extension), ctypes.POINTER(ExtensionBase)) \
            if extension is not None else None
        fr = CallFrame(ctypes.sizeof(CallFrame), ext, ctypes.pointer(self.api), None, stage,
                       table(args), table(rets), at, None)
        self._keep.append(fr)
        return fr

    def call(self, lib, name, frame):
        fn = getattr(lib, name)
        fn.restype = c_vp
        fn.argtypes = [ctypes.POINTER(CallFrame)]
        return fn(ctypes.byref(frame))
