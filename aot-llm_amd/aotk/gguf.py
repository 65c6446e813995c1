"""GGUF ingestion: the parser and writer of crates/aot-gguf/src/lib.rs and the
model table of crates/aot-codegen/src/model.rs:194-440 (`ModelSpec::from_gguf`).

`open_model(path)` maps a GGUF file, reads its hyper-parameters and tensor
table into an `aotk_model_spec` whose tensor offsets are relative to the
tensor-data section, and hands that section (memory-mapped, not copied) to
`aotk_model_load`, which uploads it to HBM once: the same bytes aot-codegen
embeds with `.incbin` (emit.rs:707-795). `GgufWriter` builds files in memory
(lib.rs:392-511); `config_gguf` emits a config model as a GGUF file.
"""
import ctypes as C
import mmap
import struct

from . import abi

GGUF_MAGIC = 0x46554747  # "GGUF" little-endian (lib.rs:21)
DEFAULT_ALIGNMENT = 32   # lib.rs:23

# ggml_type id -> (name, block size, type size) (types.rs:9-127)
GGML_TYPES = {
    0: ("f32", 1, 4), 1: ("f16", 1, 2), 2: ("q4_0", 32, 18), 3: ("q4_1", 32, 20), 6: ("q5_0", 32, 22),
    7: ("q5_1", 32, 24), 8: ("q8_0", 32, 34), 9: ("q8_1", 32, 36), 10: ("q2_K", 256, 84), 11: ("q3_K", 256, 110),
    12: ("q4_K", 256, 144), 13: ("q5_K", 256, 176), 14: ("q6_K", 256, 210), 15: ("q8_K", 256, 292),
    16: ("iq2_xxs", 256, 66), 17: ("iq2_xs", 256, 74), 18: ("iq3_xxs", 256, 98), 19: ("iq1_s", 256, 50),
    20: ("iq4_nl", 32, 18), 21: ("iq3_s", 256, 110), 22: ("iq2_s", 256, 82), 23: ("iq4_xs", 256, 136),
    24: ("i8", 1, 1), 25: ("i16", 1, 2), 26: ("i32", 1, 4), 27: ("i64", 1, 8), 28: ("f64", 1, 8),
    29: ("iq1_m", 256, 56), 30: ("bf16", 1, 2), 34: ("tq1_0", 256, 54), 35: ("tq2_0", 256, 66),
}
# the kinds the hot path runs (model.rs tensor_spec / Kind::from_ggml)
GGML_TO_KIND = {0: abi.F32, 1: abi.F16, 30: abi.BF16, 2: abi.Q4_0, 6: abi.Q5_0, 8: abi.Q8_0,
                12: abi.Q4_K, 13: abi.Q5_K, 14: abi.Q6_K}
KIND_TO_GGML = {k: t for t, k in GGML_TO_KIND.items()}

# metadata value types (lib.rs:355-379)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", U64: "<Q", I64: "<q",
           F64: "<d"}


class GgufError(ValueError):
    """A malformed or unsupported file (lib.rs GgufError / model.rs bail!)."""


class Meta:
    """One metadata value with its GGUF type (MetaValue)."""

    __slots__ = ("ty", "value")

    def __init__(self, ty, value):
        self.ty, self.value = ty, value

    def as_u64(self):  # lib.rs:45-58: any integer or bool, lossy
        if self.ty in (U8, I8, U16, I16, U32, I32, U64, I64, BOOL):
            return int(self.value) & 0xFFFFFFFFFFFFFFFF
        return None

    def as_f64(self):  # :61-67
        if self.ty in (F32, F64):
            return float(self.value)
        u = self.as_u64()
        return None if u is None else float(u)

    def __eq__(self, other):
        return isinstance(other, Meta) and self.ty == other.ty and self.value == other.value

    def __repr__(self):
        return f"Meta({self.ty}, {self.value!r})"


class TensorInfo:
    """A tensor descriptor (lib.rs:110-140); dims in ggml order (innermost first)."""

    def __init__(self, name, dims, ty, offset):
        self.name, self.dims, self.ty, self.offset = name, list(dims), ty, offset

    def n_elements(self):
        n = 1
        for d in self.dims:
            n *= d
        return n

    def n_bytes(self):
        _, block, size = GGML_TYPES[self.ty]
        return self.n_elements() // block * size

    def cols(self):
        return self.dims[0] if self.dims else 1

    def rows(self):
        n = 1
        for d in self.dims[1:]:
            n *= d
        return n


class _Reader:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n, what):
        end = self.pos + n
        if end > len(self.buf):
            raise GgufError(f"file truncated while reading {what} at offset {self.pos}")
        s = self.buf[self.pos:end]
        self.pos = end
        return s

    def scalar(self, fmt, what):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt), what))[0]

    def string(self, what):
        n = self.scalar("<Q", what)
        start = self.pos
        try:
            return bytes(self.take(n, what)).decode("utf-8")
        except UnicodeDecodeError:
            raise GgufError(f"invalid UTF-8 in string at offset {start}") from None

    def value(self, vt):
        w = "metadata value"
        if vt in _SCALAR:
            return Meta(vt, self.scalar(_SCALAR[vt], w))
        if vt == BOOL:
            return Meta(BOOL, self.scalar("<B", w) != 0)
        if vt == STRING:
            return Meta(STRING, self.string(w))
        if vt == ARRAY:
            et = self.scalar("<I", "array element type")
            n = self.scalar("<Q", "array length")
            if n > len(self.buf):  # guard before allocating (lib.rs:367-370)
                raise GgufError(f"file truncated while reading array at offset {self.pos}")
            return Meta(ARRAY, [self.value(et) for _ in range(n)])
        raise GgufError(f"unknown metadata value type {vt}")


class GgufFile:
    """Header, metadata and tensor table (GgufFile::parse, lib.rs:160-222)."""

    def __init__(self, buf, file_len=None):
        file_len = len(buf) if file_len is None else file_len
        r = _Reader(memoryview(buf))
        magic = r.scalar("<I", "magic")
        if magic != GGUF_MAGIC:
            raise GgufError(f'bad magic: expected "GGUF", found {magic:#010x}')
        self.version = r.scalar("<I", "version")
        if self.version not in (2, 3):
            raise GgufError(f"unsupported GGUF version {self.version} (supported: 2, 3)")
        n_tensors = r.scalar("<Q", "tensor count")
        n_kv = r.scalar("<Q", "metadata count")
        self.metadata = []
        self.meta = {}
        for _ in range(n_kv):
            key = r.string("metadata key")
            vt = r.scalar("<I", "metadata value type")
            v = r.value(vt)
            self.meta[key] = v
            self.metadata.append((key, v))
        a = self.meta.get("general.alignment")
        self.alignment = a.as_u64() if a is not None and a.as_u64() is not None else DEFAULT_ALIGNMENT
        if self.alignment == 0 or self.alignment & (self.alignment - 1):
            raise GgufError(f"invalid alignment {self.alignment} (must be a power of two)")
        self.tensors = []
        self.by_name = {}
        for _ in range(n_tensors):
            name = r.string("tensor name")
            n_dims = r.scalar("<I", "tensor n_dims")
            if n_dims > 4:
                raise GgufError(f'tensor "{name}" has {n_dims} dimensions (max 4)')
            dims = [r.scalar("<Q", "tensor dim") for _ in range(n_dims)]
            ty = r.scalar("<I", "tensor type")
            if ty not in GGML_TYPES:
                raise GgufError(f'unknown tensor type id {ty} for tensor "{name}"')
            off = r.scalar("<Q", "tensor offset")
            self.by_name[name] = len(self.tensors)
            self.tensors.append(TensorInfo(name, dims, ty, off))
        self.data_offset = (r.pos + self.alignment - 1) // self.alignment * self.alignment
        for t in self.tensors:
            start = self.data_offset + t.offset
            end = start + t.n_bytes()
            if end > file_len:
                raise GgufError(f'tensor "{t.name}" data range [{start}, {end}) exceeds file size {file_len}')

    def get(self, key):
        return self.meta.get(key)

    def _require(self, key):
        v = self.meta.get(key)
        if v is None:
            raise GgufError(f'metadata key "{key}" not found')
        return v

    def get_str(self, key):
        v = self._require(key)
        if v.ty != STRING:
            raise GgufError(f'metadata key "{key}" has unexpected type (expected string)')
        return v.value

    def get_u64(self, key):
        u = self._require(key).as_u64()
        if u is None:
            raise GgufError(f'metadata key "{key}" has unexpected type (expected integer)')
        return u

    def get_f64(self, key):
        f = self._require(key).as_f64()
        if f is None:
            raise GgufError(f'metadata key "{key}" has unexpected type (expected number)')
        return f

    def get_array(self, key):
        v = self._require(key)
        if v.ty != ARRAY:
            raise GgufError(f'metadata key "{key}" has unexpected type (expected array)')
        return v.value

    def architecture(self):
        return self.get_str("general.architecture")

    def tensor(self, name):
        i = self.by_name.get(name)
        return None if i is None else self.tensors[i]

    def require_tensor(self, name):
        t = self.tensor(name)
        if t is None:
            raise GgufError(f'tensor "{name}" not found')
        return t

    def data_len(self):
        return max((t.offset + t.n_bytes() for t in self.tensors), default=0)

    def n_params(self):
        return sum(t.n_elements() for t in self.tensors)


class GgufWriter:
    """Incremental GGUF v3 writer (lib.rs:392-447)."""

    def __init__(self, alignment=DEFAULT_ALIGNMENT):
        self.kvs, self.tensors, self.alignment = [], [], alignment

    def kv(self, key, value):
        assert isinstance(value, Meta)
        self.kvs.append((key, value))
        return self

    def tensor(self, name, dims, ty, data):
        t = TensorInfo(name, dims, ty, 0)
        data = bytes(data)
        assert t.n_bytes() == len(data), f"tensor {name}: data size mismatch"
        self.tensors.append((name, list(dims), ty, data))
        return self

    @staticmethod
    def _string(out, s):
        b = s.encode("utf-8")
        out += struct.pack("<Q", len(b)) + b

    def _value(self, out, v, with_type=True):
        if with_type:
            out += struct.pack("<I", v.ty)
        if v.ty in _SCALAR:
            out += struct.pack(_SCALAR[v.ty], v.value)
        elif v.ty == BOOL:
            out += struct.pack("<B", 1 if v.value else 0)
        elif v.ty == STRING:
            self._string(out, v.value)
        elif v.ty == ARRAY:
            et = v.value[0].ty if v.value else U32  # lib.rs:488
            out += struct.pack("<IQ", et, len(v.value))
            for e in v.value:
                assert e.ty == et, "heterogeneous GGUF array"
                self._value(out, e, False)
        else:
            raise GgufError(f"unknown metadata value type {v.ty}")

    def finish(self):
        a = self.alignment
        out = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(self.tensors), len(self.kvs)))
        for k, v in self.kvs:
            self._string(out, k)
            self._value(out, v)
        off = 0
        for name, dims, ty, data in self.tensors:
            self._string(out, name)
            out += struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", ty, off)
            off = (off + len(data) + a - 1) // a * a
        out += b"\x00" * ((-len(out)) % a)
        for _, _, _, data in self.tensors:
            out += data
            out += b"\x00" * ((-len(out)) % a)
        return bytes(out)


# ---------------------------------------------------------------- model table
# model.rs:183-192 (plus the fused q/k/v and gate/up of Phi-3)
ARCH_FLAGS = {
    "llama": dict(),
    "qwen2": dict(rope_neox=1, qkv_bias=1),
    "qwen3": dict(rope_neox=1, qk_norm=1),
    "phi3": dict(rope_neox=1, fused_qkv=1, fused_gate_up=1),
    "gemma3": dict(rope_neox=1, qk_norm=1, embd_scale=1, post_norms=1, gelu=1, swa_pattern=6),
}


class GgufSpec:
    """`ModelSpec::from_gguf` (model.rs:283-440) as an aotk_model_spec with
    offsets relative to the tensor-data section; the same attributes as
    configs.Spec (`spec`, `d`, `layers`, `blob_len`, `ptr()`)."""

    def __init__(self, g):
        arch = g.architecture()
        if arch not in ARCH_FLAGS:
            raise GgufError(f'unsupported architecture "{arch}": supported are ' +
                            ", ".join(f'"{a}"' for a in ARCH_FLAGS))
        flags = ARCH_FLAGS[arch]
        self.arch, self.warnings = arch, []
        if g.tensor("rope_factors_long.weight") or g.tensor("rope_factors_short.weight"):
            raise GgufError("this model uses LongRoPE scaling (rope_factors_long/short), which is not supported")

        def k(s):
            return f"{arch}.{s}"

        def opt(getter, key, default):
            try:
                return getter(key)
            except GgufError:
                return default

        dim = g.get_u64(k("embedding_length"))
        hidden = g.get_u64(k("feed_forward_length"))
        n_layer = g.get_u64(k("block_count"))
        n_head = g.get_u64(k("attention.head_count"))
        n_kv_head = opt(g.get_u64, k("attention.head_count_kv"), n_head)
        head_dim = opt(g.get_u64, k("attention.key_length"), dim // n_head)
        rot_dim = opt(g.get_u64, k("rope.dimension_count"), head_dim)
        eps = opt(g.get_f64, k("attention.layer_norm_rms_epsilon"), 1e-5)
        rope_base = opt(g.get_f64, k("rope.freq_base"), 10000.0)
        n_ctx_train = opt(g.get_u64, k("context_length"), 2048)
        rope_scale = 1.0
        try:
            st = g.get_str(k("rope.scaling.type"))
        except GgufError:
            st = None
        if st is not None:
            factor = opt(g.get_f64, k("rope.scaling.factor"), 1.0)
            if st == "linear":
                rope_scale = factor
            elif st not in ("none", ""):
                self.warnings.append(f'rope scaling type "{st}" (factor {factor}) is not supported; positions are used unscaled')
        if n_head % n_kv_head:
            raise GgufError(f"head_count {n_head} is not a multiple of head_count_kv {n_kv_head}")
        swa_window = 0
        if flags.get("swa_pattern"):
            try:
                swa_window = g.get_u64(k("attention.sliding_window"))
            except GgufError:
                raise GgufError("sliding-window architecture without attention.sliding_window") from None
        if rot_dim > head_dim or rot_dim % 2:
            raise GgufError(f"invalid rope dimension count {rot_dim} for head_dim {head_dim}")
        tok = g.get("tokenizer.ggml.tokens")
        if tok is not None and tok.ty == ARRAY:
            vocab = len(tok.value)
        else:
            try:
                vocab = g.get_u64(k("vocab_size"))
            except GgufError:
                raise GgufError("no tokenizer.ggml.tokens and no vocab_size") from None
        q_dim, kv_dim = n_head * head_dim, n_kv_head * head_dim

        self.d = dict(dim=dim, hidden=hidden, n_layer=n_layer, n_head=n_head, n_kv_head=n_kv_head,
                      head_dim=head_dim, vocab=vocab, rot_dim=rot_dim)
        s = self.spec = abi.ModelSpec()
        for key, v in self.d.items():
            setattr(s.dims, key, v)
        s.dims.n_ctx_train = n_ctx_train
        s.dims.eps = eps
        s.dims.rope_base = rope_base
        s.dims.rope_scale = rope_scale
        s.dims.swa_window = swa_window
        s.dims.rope_base_local = 10000.0  # model.rs:350
        s.dims.rope_scale_local = 1.0
        for f in ("rope_neox", "qkv_bias", "qk_norm", "embd_scale", "post_norms", "gelu"):
            setattr(s.flags, f, flags.get(f, 0))
        s.flags.swa_pattern = flags.get("swa_pattern", 0)
        used = []

        def tspec(t):
            kind = GGML_TO_KIND.get(t.ty)
            if kind is None:
                raise GgufError(f"tensor {t.name} uses unsupported type {GGML_TYPES[t.ty][0]}; supported: "
                                "f32, f16, bf16, q4_0, q5_0, q8_0, q4_K, q5_K, q6_K")
            cols = t.cols()
            if cols % abi.BLOCK[kind]:
                raise GgufError(f"tensor {t.name}: inner dimension {cols} is not a multiple of the "
                                f"{GGML_TYPES[t.ty][0]} block size")
            x = abi.Tensor()
            x.kind, x.off, x.len, x.rows, x.cols = kind, t.offset, t.n_bytes(), t.rows(), cols
            used.append(t.name)
            return x

        def matrix(name, rows, cols):
            t = g.require_tensor(name)
            x = tspec(t)
            if x.rows != rows or x.cols != cols:
                raise GgufError(f"tensor {name}: expected shape [{cols} x {rows}] (ggml order), found {t.dims}")
            return x

        def vector(name, n):
            t = g.require_tensor(name)
            x = tspec(t)
            if x.kind != abi.F32:
                raise GgufError(f"tensor {name}: norm weights must be f32, found {GGML_TYPES[t.ty][0]}")
            if t.n_elements() != n:
                raise GgufError(f"tensor {name}: expected {n} elements, found {t.n_elements()}")
            return x

        def rows_view(x, row0, rows):  # model.rs:257-262
            rb = x.len // x.rows
            y = abi.Tensor()
            y.kind, y.off, y.len, y.rows, y.cols = x.kind, x.off + row0 * rb, rows * rb, rows, x.cols
            return y

        def none():
            t = abi.Tensor()
            t.kind = abi.NONE
            return t

        s.token_embd = matrix("token_embd.weight", vocab, dim)
        s.output_norm = vector("output_norm.weight", dim)
        s.output = matrix("output.weight", vocab, dim) if g.tensor("output.weight") else none()
        rf = g.tensor("rope_freqs.weight")
        if rf is not None:
            x = tspec(rf)
            if x.kind != abi.F32 or rf.n_elements() != rot_dim // 2:
                raise GgufError(f"rope_freqs.weight must be f32[{rot_dim // 2}]")
            s.rope_freqs = x
        else:
            s.rope_freqs = none()
        self.layers = (abi.Layer * n_layer)()
        for i in range(n_layer):
            L = self.layers[i]

            def p(n):
                return f"blk.{i}.{n}.weight"

            def b(n):
                return f"blk.{i}.{n}.bias"

            if flags.get("qkv_bias"):
                L.bq, L.bk, L.bv = vector(b("attn_q"), q_dim), vector(b("attn_k"), kv_dim), vector(b("attn_v"), kv_dim)
            else:
                L.bq, L.bk, L.bv = none(), none(), none()
            if flags.get("qk_norm"):
                L.q_norm, L.k_norm = vector(p("attn_q_norm"), head_dim), vector(p("attn_k_norm"), head_dim)
            else:
                L.q_norm, L.k_norm = none(), none()
            if flags.get("post_norms"):
                L.attn_post_norm, L.ffn_post_norm = vector(p("post_attention_norm"), dim), vector(p("post_ffw_norm"), dim)
            else:
                L.attn_post_norm, L.ffn_post_norm = none(), none()
            pat = flags.get("swa_pattern", 0)
            L.local_attn = 1 if pat > 0 and (i + 1) % pat != 0 else 0
            if flags.get("fused_qkv"):
                qkv = matrix(p("attn_qkv"), q_dim + 2 * kv_dim, dim)
                L.wq, L.wk, L.wv = rows_view(qkv, 0, q_dim), rows_view(qkv, q_dim, kv_dim), rows_view(qkv, q_dim + kv_dim, kv_dim)
            else:
                L.wq, L.wk, L.wv = matrix(p("attn_q"), q_dim, dim), matrix(p("attn_k"), kv_dim, dim), matrix(p("attn_v"), kv_dim, dim)
            if flags.get("fused_gate_up"):
                gu = matrix(p("ffn_up"), 2 * hidden, dim)
                L.gate, L.up = rows_view(gu, 0, hidden), rows_view(gu, hidden, hidden)
            else:
                L.gate, L.up = matrix(p("ffn_gate"), hidden, dim), matrix(p("ffn_up"), hidden, dim)
            L.attn_norm = vector(p("attn_norm"), dim)
            L.wo = matrix(p("attn_output"), dim, q_dim)
            L.ffn_norm = vector(p("ffn_norm"), dim)
            L.down = matrix(p("ffn_down"), dim, hidden)
        s.layers = C.cast(self.layers, C.POINTER(abi.Layer))
        # tensors the graph does not read: ignored, except biases (model.rs:394-425)
        unused = sorted(set(t.name for t in g.tensors) - set(used))
        for n in unused:
            if "bias" in n:
                raise GgufError(f"tensor {n}: bias tensors are not supported by the {arch} graph")
        if unused:
            self.warnings.append(f"{len(g.tensors)} tensors in file, {len(g.tensors) - len(unused)} used by the graph "
                                 f"(unused: {', '.join(unused[:5])})")
        self.blob_len = g.data_len()
        self.data_offset = g.data_offset

    def ptr(self):
        return C.pointer(self.spec)


def open_file(path):
    """Map `path` and parse it: (GgufFile, memoryview of the whole file)."""
    f = open(path, "rb")
    try:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    finally:
        f.close()
    return GgufFile(mm, len(mm)), mm


def open_model(path):
    """A GGUF file as (GgufSpec, tensor-data section bytes) ready for
    `aotk.Model(spec, data)`."""
    g, mm = open_file(path)
    spec = GgufSpec(g)
    data = memoryview(mm)[g.data_offset:g.data_offset + g.data_len()]
    return spec, data


def config_gguf(spec, blob, arch, fuse=False, name="aotk-config"):
    """Emit a built config (configs.Spec) with its tensor blob as a GGUF v3
    file (bytes): llama.cpp's metadata keys for `arch`, the tensors named
    like configs.Spec.tensors in blob order. fuse=True writes Phi-3's fused
    attn_qkv and ffn_up (gate rows first), which needs matching kinds."""
    d = spec.d
    sd = spec.spec.dims
    w = GgufWriter()
    w.kv("general.architecture", Meta(STRING, arch))
    w.kv("general.name", Meta(STRING, name))
    w.kv(f"{arch}.embedding_length", Meta(U32, d["dim"]))
    w.kv(f"{arch}.feed_forward_length", Meta(U32, d["hidden"]))
    w.kv(f"{arch}.block_count", Meta(U32, d["n_layer"]))
    w.kv(f"{arch}.attention.head_count", Meta(U32, d["n_head"]))
    w.kv(f"{arch}.attention.head_count_kv", Meta(U32, d["n_kv_head"]))
    w.kv(f"{arch}.attention.key_length", Meta(U32, d["head_dim"]))
    w.kv(f"{arch}.rope.dimension_count", Meta(U32, d["rot_dim"]))
    w.kv(f"{arch}.attention.layer_norm_rms_epsilon", Meta(F32, float(sd.eps)))
    w.kv(f"{arch}.rope.freq_base", Meta(F32, float(sd.rope_base)))
    w.kv(f"{arch}.context_length", Meta(U32, int(sd.n_ctx_train)))
    if float(sd.rope_scale) != 1.0:
        w.kv(f"{arch}.rope.scaling.type", Meta(STRING, "linear"))
        w.kv(f"{arch}.rope.scaling.factor", Meta(F32, float(sd.rope_scale)))
    if int(sd.swa_window):
        w.kv(f"{arch}.attention.sliding_window", Meta(U32, int(sd.swa_window)))
    w.kv(f"{arch}.vocab_size", Meta(U32, d["vocab"]))
    blob = bytes(blob)
    tensors = list(spec.tensors)  # (name, kind, rows, cols, off, len)
    if fuse:
        by = {t[0]: t for t in tensors}
        out = []
        for t in tensors:
            nm = t[0]
            if nm.endswith(("attn_k", "attn_v", "ffn_gate")):
                continue
            if nm.endswith("attn_q") or nm.endswith("ffn_up"):
                pre = nm.rsplit(".", 1)[0]
                parts = [by[pre + ".attn_q"], by[pre + ".attn_k"], by[pre + ".attn_v"]] if nm.endswith("attn_q") \
                    else [by[pre + ".ffn_gate"], by[pre + ".ffn_up"]]
                if len(set(x[1] for x in parts)) != 1:
                    raise GgufError(f"{pre}: fused tensors need one kind")
                data = b"".join(blob[x[4]:x[4] + x[5]] for x in parts)
                rows = sum(x[2] for x in parts)
                out.append((pre + (".attn_qkv" if nm.endswith("attn_q") else ".ffn_up"), parts[0][1], rows, parts[0][3], data))
            else:
                out.append((nm, t[1], t[2], t[3], blob[t[4]:t[4] + t[5]]))
    else:
        out = [(t[0], t[1], t[2], t[3], blob[t[4]:t[4] + t[5]]) for t in tensors]
    for nm, kind, rows, cols, data in out:
        gname = nm if nm.endswith(".bias") else nm + ".weight"
        dims = [cols] if rows == 1 else [cols, rows]
        w.tensor(gname, dims, KIND_TO_GGML[kind], data)
    return w.finish()
