"""Python mirror of ltx-weights' store API over include/ltxw_store.h.

`WeightStore`, `LoraFile`, `KeyMap`, `MergeReport` and `Scope` keep the names,
argument meaning and error behaviour of the reference crate
(crates/ltx-weights/src/{store,lora,key_map,scope}.rs): the same keys come out
of `open`, `merge_lora` reports and rejects the same cases, and `read`
returns the same f32 values (computed on the device). `materialize_bf16` is
the added entry point that leaves dequantised + merged bf16 tensors in HBM.
"""
import ctypes

import numpy as np

from . import _dlpack
from . import _native as N

DTYPE_NAMES = ["BOOL", "U8", "I8", "F8_E5M2", "F8_E4M3", "I16", "U16", "F16", "BF16", "I32", "U32",
               "F32", "F64", "I64", "U64", "F8_E8M0", "F4", "F6_E2M3", "F6_E3M2", "C64"]
MAT_SCALE_FIRST = 1
MAT_EXACT = 2
MAT_ROW_SCALES = 4
MAT_MFMA = 8
_MAX_DIMS = 16


def _s(x):
    return x.decode("utf-8") if x is not None else None


def _info(fn, handle, name):
    dt, nd = ctypes.c_int32(), ctypes.c_int32()
    dims = (ctypes.c_int64 * _MAX_DIMS)()
    N.check_store(fn(handle, name.encode(), ctypes.byref(dt), ctypes.byref(nd), dims, _MAX_DIMS))
    return DTYPE_NAMES[dt.value], tuple(int(dims[k]) for k in range(min(nd.value, _MAX_DIMS)))


class KeyMap:
    """Ordered key rules applied at open (src/key_map.rs:30-86, apply_key at :237-268)."""

    REQUIRE_ANY_PREFIX, REPLACE, DROP_PREFIX, DROP_SUFFIX, RENAME_EXACT = 0, 1, 2, 3, 4
    SPLIT_QKV, FOLD_GATES, SYNTH_ZERO_TYPE_EMB = 5, 6, 7

    def __init__(self, rules=()):
        self.rules = [(int(k), [str(x) for x in strs]) for k, strs in rules]

    @classmethod
    def identity(cls):
        return cls()

    @classmethod
    def transformer(cls):
        """`KeyMap::transformer` (src/key_map.rs:101-112)."""
        return cls([(cls.REQUIRE_ANY_PREFIX, ["model.diffusion_model."]),
                    (cls.REPLACE, ["model.diffusion_model.", ""])])

    @classmethod
    def video_encoder(cls):
        """`KeyMap::video_encoder` (src/key_map.rs:123-146)."""
        return cls([(cls.REQUIRE_ANY_PREFIX, ["vae.encoder.", "vae.per_channel_statistics.", "encoder.",
                                              "per_channel_statistics."]),
                    (cls.REPLACE, ["vae.encoder.", ""]),
                    (cls.REPLACE, ["vae.per_channel_statistics.", "per_channel_statistics."]),
                    (cls.REPLACE, ["encoder.", ""])])

    @classmethod
    def video_decoder(cls):
        """`KeyMap::video_decoder` (src/key_map.rs:167-208), value transforms included."""
        return cls([(cls.REQUIRE_ANY_PREFIX, ["vae.decoder.", "decoder.", "vae.per_channel_statistics.",
                                              "per_channel_statistics."]),
                    (cls.REPLACE, ["vae.decoder.", ""]),
                    (cls.REPLACE, ["decoder.", ""]),
                    (cls.REPLACE, ["vae.per_channel_statistics.", "per_channel_statistics."]),
                    (cls.RENAME_EXACT, ["t_embedder.mlp.0.", "t_embedder.timestep_embedder.linear_1."]),
                    (cls.RENAME_EXACT, ["t_embedder.mlp.2.", "t_embedder.timestep_embedder.linear_2."]),
                    (cls.DROP_PREFIX, ["coarse_"]),
                    (cls.FOLD_GATES, []),
                    (cls.SPLIT_QKV, []),
                    (cls.SYNTH_ZERO_TYPE_EMB, [])])

    def _c(self):
        keep = []
        arr = (N.KeyRule * max(1, len(self.rules)))()
        for k, (kind, strs) in enumerate(self.rules):
            enc = (ctypes.c_char_p * max(1, len(strs)))(*[x.encode() for x in strs])
            keep.append(enc)
            arr[k] = N.KeyRule(kind, len(strs), ctypes.cast(enc, ctypes.POINTER(ctypes.c_char_p)))
        return arr, keep


class MergeReport:
    """`MergeReport` (src/lora.rs:157-170); key lists in byte order."""

    def __init__(self, matched_keys, unmatched_lora_keys):
        self.matched_keys = matched_keys
        self.unmatched_lora_keys = unmatched_lora_keys

    def __repr__(self):
        return f"MergeReport(matched={len(self.matched_keys)}, unmatched={len(self.unmatched_lora_keys)})"


class LoraFile:
    """`LoraFile` (src/lora.rs:43-152)."""

    def __init__(self, handle):
        self.h = handle

    @classmethod
    def open(cls, path):
        h = ctypes.c_void_p()
        N.check_store(N.lib().ltxw_lora_open(str(path).encode(), ctypes.byref(h)))
        return cls(h)

    def close(self):
        if self.h:
            N.lib().ltxw_lora_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()

    def tensor_names(self):
        L = N.lib()
        return [_s(L.ltxw_lora_tensor_name(self.h, k)) for k in range(L.ltxw_lora_n_tensors(self.h))]

    def tensor_info(self, name):
        """(dtype name, shape), or None when absent."""
        try:
            return _info(N.lib().ltxw_lora_tensor_info, self.h, name)
        except N.MissingKey:
            return None

    def metadata(self, key):
        return _s(N.lib().ltxw_lora_metadata(self.h, key.encode()))

    def ic_layout(self):
        """(reference_downscale_factor, reference_temporal_scale_factor)."""
        d, t = ctypes.c_uint32(), ctypes.c_uint32()
        N.check_store(N.lib().ltxw_lora_ic_layout(self.h, ctypes.byref(d), ctypes.byref(t)))
        return d.value, t.value

    def read_f32(self, name):
        """(shape, f32 array), or None when the name is absent (src/lora.rs:124-146)."""
        info = self.tensor_info(name)
        if info is None:
            return None
        shape = info[1]
        out = np.empty(int(np.prod(shape, dtype=np.int64)), dtype=np.float32)
        N.check_store(N.lib().ltxw_lora_read_f32(self.h, name.encode(), out.ctypes.data, out.size))
        return list(shape), out


class DeviceTensor:
    """A materialised tensor in HBM (bf16 or f32, row-major), owned by `ctx`."""

    def __init__(self, ctx, ptr, shape, out_dtype):
        self.ctx, self.ptr, self.shape, self.out_dtype = ctx, ptr, tuple(shape), out_dtype

    @property
    def numel(self):
        return int(np.prod(self.shape, dtype=np.int64))

    @property
    def nbytes(self):
        return self.numel * (2 if self.out_dtype == N.OUT_BF16 else 4)

    def to_numpy(self):
        """bf16 as uint16 bit patterns, or f32."""
        out = np.empty(self.shape, dtype=np.uint16 if self.out_dtype == N.OUT_BF16 else np.float32)
        if self.numel:
            self.ctx.download(self.ptr, out)
        return out

    def free(self):
        if self.ptr:
            self.ctx.free(self.ptr)
            self.ptr = None

    # DLPack export: the tensor's HBM, no copy, for any DLPack consumer in the
    # process that uses the same HIP runtime. The capsule does not own the
    # memory: keep this DeviceTensor alive (and unfreed) while it is in use.
    def __dlpack_device__(self):
        return (_dlpack.KDL_ROCM, self.ctx.device)

    def __dlpack__(self, stream=None):
        if not self.ptr and self.numel:
            raise N.InvalidArgument("tensor was freed")
        self.ctx.synchronize()  # the data is complete before any consumer stream uses it
        return _dlpack.capsule(self.ptr, self.shape, self.out_dtype == N.OUT_BF16, self.ctx.device, owner=self)


class WeightStore:
    """`WeightStore` (src/store.rs:89-640) with the device materialisation path."""

    def __init__(self, handle):
        self.h = handle

    @classmethod
    def open(cls, paths, key_map=None):
        if isinstance(paths, (str, bytes)) or hasattr(paths, "__fspath__"):
            paths = [paths]
        km = key_map or KeyMap.identity()
        enc = [str(p).encode() for p in paths]
        parr = (ctypes.c_char_p * max(1, len(enc)))(*enc)
        rules, keep = km._c()
        h = ctypes.c_void_p()
        N.check_store(N.lib().ltxw_store_open(parr, len(enc), rules, len(km.rules), ctypes.byref(h)))
        del keep
        return cls(h)

    def close(self):
        if self.h:
            N.lib().ltxw_store_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()

    def keys(self):
        L = N.lib()
        return [_s(L.ltxw_store_key(self.h, k)) for k in range(L.ltxw_store_n_keys(self.h))]

    def contains(self, key):
        return bool(N.lib().ltxw_store_contains(self.h, key.encode()))

    def shape(self, key):
        return list(_info(N.lib().ltxw_store_tensor_info, self.h, key)[1])

    def dtype(self, key):
        return _info(N.lib().ltxw_store_tensor_info, self.h, key)[0]

    def metadata(self, key):
        return _s(N.lib().ltxw_store_metadata(self.h, key.encode()))

    def merge_lora(self, lora, strength):
        rep = ctypes.c_void_p()
        N.check_store(N.lib().ltxw_store_merge_lora(self.h, lora.h, ctypes.c_float(strength), ctypes.byref(rep)))
        L = N.lib()
        try:
            matched = [_s(L.ltxw_report_matched(rep, k)) for k in range(L.ltxw_report_n_matched(rep))]
            unmatched = [_s(L.ltxw_report_unmatched(rep, k)) for k in range(L.ltxw_report_n_unmatched(rep))]
        finally:
            L.ltxw_report_free(rep)
        return MergeReport(matched, unmatched)

    def deltas(self, key):
        """[(rank, coeff)] merged into `key`, in application order."""
        L = N.lib()
        out = []
        for k in range(L.ltxw_store_n_deltas(self.h, key.encode())):
            r, c = ctypes.c_int32(), ctypes.c_float()
            N.check_store(L.ltxw_store_delta(self.h, key.encode(), k, ctypes.byref(r), ctypes.byref(c)))
            out.append((r.value, c.value))
        return out

    def read(self, key, ctx, flags=0):
        """`read` (src/store.rs:479-521) on the device: (shape, f32 array),
        bit-identical to the reference's unless `flags` opts into an
        extension (MAT_ROW_SCALES, MAT_MFMA)."""
        shape = self.shape(key)
        out = np.empty(int(np.prod(shape, dtype=np.int64)), dtype=np.float32)
        N.check_store(N.lib().ltxw_store_read(self.h, ctx.h, key.encode(), flags, out.ctypes.data, out.size))
        return shape, out.reshape(shape)

    def materialize(self, ctx, keys, outs, out_dtype=N.OUT_BF16, flags=0):
        """Into caller-owned device pointers outs[k] (numel(keys[k]) elements
        each). Per-row scales; LoRA deltas in the reference's operation order
        (bit-identical) unless `flags` has MAT_MFMA."""
        karr = (ctypes.c_char_p * max(1, len(keys)))(*[k.encode() for k in keys])
        oarr = (ctypes.c_void_p * max(1, len(outs)))(*outs)
        N.check_store(N.lib().ltxw_store_materialize(self.h, ctx.h, karr, len(keys), out_dtype, flags, oarr))

    def materialize_bf16(self, ctx, keys=None, flags=0):
        """{key: DeviceTensor} of bf16 tensors in HBM (every visible key by default)."""
        keys = self.keys() if keys is None else list(keys)
        shapes = [self.shape(k) for k in keys]
        outs = []
        try:
            for sh in shapes:
                n = int(np.prod(sh, dtype=np.int64))
                outs.append(ctx.alloc(2 * n) if n else None)
            self.materialize(ctx, keys, outs, N.OUT_BF16, flags)
        except Exception:
            for p in outs:
                if p:
                    ctx.free(p)
            raise
        return {k: DeviceTensor(ctx, p, sh, N.OUT_BF16) for k, p, sh in zip(keys, outs, shapes)}

    def scope(self, prefix):
        return Scope(self, prefix)


class Scope:
    """`Scope` (src/scope.rs:13-92): a dot-joined key prefix over a store."""

    def __init__(self, store, prefix):
        self.store, self.prefix = store, prefix

    def scope(self, child):
        return Scope(self.store, child if not self.prefix else f"{self.prefix}.{child}")

    def full_key(self, name):
        return name if not self.prefix else f"{self.prefix}.{name}"

    def contains(self, name):
        return self.store.contains(self.full_key(name))

    def tensor(self, name, ctx):
        """(shape, f32 array) of `read` at the scoped key."""
        return self.store.read(self.full_key(name), ctx)

    def optional(self, name, ctx):
        return self.tensor(name, ctx) if self.contains(name) else None
