"""ctypes binding of libsa_amd.so, the gfx950 streaming-attention library.

The directory name carries a hyphen, so load it by path:

    import importlib.util, pathlib
    spec = importlib.util.spec_from_file_location(
        "streaming_attention_amd", "streaming-attention_amd/__init__.py",
        submodule_search_locations=["streaming-attention_amd"])

Device buffers are torch tensors (torch is used for device memory and streams
only); every call goes through the C ABI declared in include/sa_amd.h.  There is
no fallback: if the library is missing, `lib()` raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "lib" / "libsa_amd.so"

SA_OK = 0
SA_EINVAL = -1
SA_ENOMEM = -2
SA_EFULL = -3
SA_EHIP = -4
SA_ERANGE = -5
SA_EIO = -6
SA_DTYPE_F32 = 0
SA_DTYPE_BF16 = 1
PAGE_TOKENS = 64

_STATUS_NAMES = {0: "SA_OK", -1: "SA_EINVAL", -2: "SA_ENOMEM", -3: "SA_EFULL",
                 -4: "SA_EHIP", -5: "SA_ERANGE", -6: "SA_EIO"}


class SaError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{_STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


class KvDesc(C.Structure):
    _fields_ = [("num_layers", C.c_int), ("num_kv_heads", C.c_int), ("head_dim", C.c_int),
                ("max_seqs", C.c_int), ("max_pages_per_seq", C.c_int), ("num_pages", C.c_int),
                ("kv_dtype", C.c_int)]


_P = C.c_void_p
_I = C.c_int
_F = C.c_float
_SZ = C.c_size_t

class Qwen3Desc(C.Structure):
    _fields_ = [("num_layers", C.c_int), ("hidden", C.c_int), ("intermediate", C.c_int),
                ("vocab", C.c_int), ("n_q_heads", C.c_int), ("n_kv_heads", C.c_int),
                ("head_dim", C.c_int), ("max_pos", C.c_int), ("rms_eps", C.c_float),
                ("rope_theta", C.c_float)]


# name -> (restype, argtypes); mirrors include/sa_amd.h and include/sa_qwen3.h
SIGNATURES = {
    "sa_last_error": (C.c_char_p, []),
    "sa_stream_attn_ws_bytes": (_SZ, [_I, _I]),
    "sa_stream_attn_f32": (_I, [_P, _P, _P, _I, _I, _I, _F, _P, _P, _SZ, _P]),
    "sa_stream_attn_f32_noalloc": (_I, [_P, _P, _P, _I, _I, _I, _F, _P, _P]),
    "sa_decode_dense_ws_bytes": (_SZ, [_I, _I, _I, _I]),
    "sa_decode_dense_f32": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _SZ, _P]),
    "sa_kvcache_create": (_I, [C.POINTER(KvDesc), C.POINTER(_P)]),
    "sa_kvcache_destroy": (_I, [_P]),
    "sa_kvcache_reset": (_I, [_P, _P]),
    "sa_kvcache_reserve": (_I, [_P, _I, _I, _P]),
    "sa_kvcache_set_pages": (_I, [_P, _I, _P, _I, _P]),
    "sa_kvcache_set_len": (_I, [_P, _I, _I, _P]),
    "sa_kvcache_len": (_I, [_P, _I]),
    "sa_kvcache_capacity": (_I, [_P, _I]),
    "sa_kvcache_commit": (_I, [_P, _P, _I, _I, _P]),
    "sa_kvcache_k_pool": (_P, [_P, _I]),
    "sa_kvcache_v_pool": (_P, [_P, _I]),
    "sa_kvcache_block_table": (_P, [_P]),
    "sa_kvcache_seq_lens": (_P, [_P]),
    "sa_kvcache_bytes": (_SZ, [_P]),
    "sa_kvcache_get_desc": (_I, [_P, C.POINTER(KvDesc)]),
    "sa_rope_table_init": (_I, [_P, _P, _I, _I, _F, _P]),
    "sa_qknorm_rope_append": (_I, [_P, _I, _P, _P, _P, _I, _I, _P, _I, _P, _P, _F, _P, _P, _I,
                                   _P, _P]),
    "sa_qk_norm_rope": (_I, [_P, _I, _I, _P, _P, _F, _P, _P, _I, _P, _P]),
    "sa_qk_norm_rope_ex": (_I, [_P, _I, _I, _P, _P, _F, _I, _P, _P, _I, _P, _P]),
    "sa_linear_f32": (_I, [_P, _I, _I, _P, _I, _P, _P, _P]),
    "sa_rms_norm_f32": (_I, [_P, _I, _I, _P, _F, _P, _P]),
    "sa_swiglu_f32": (_I, [_P, _P, _SZ, _P, _P]),
    "sa_axpby_f32": (_I, [_P, _F, _P, _F, _SZ, _P, _P]),
    "sa_paged_decode_ws_bytes": (_SZ, [_P, _I, _I]),
    "sa_paged_decode": (_I, [_P, _I, _P, _I, _P, _I, _I, _F, _P, _P, _SZ, _P]),
    "sa_append_decode_partials": (_I, [_P, _I, _P, _I, _I, _P, _I, _P, _P, _F, _P, _P, _I, _F, _P, _P, _P,
                                       _SZ, _I, _P]),
    "sa_kvcache_gather": (_I, [_P, _I, _I, _I, _P, _P, _P]),
    "sa_append_decode": (_I, [_P, _I, _P, _P, _P, _I, _P, _I, _P, _P, _F, _P, _P, _I, _F, _P, _P, _P, _SZ,
                              _I, _P]),
    "sa_prefill_causal": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _P]),
    "sa_prefill_causal_strided": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _F, _P, _P]),
    "sa_prefill_causal_ws_bytes": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "sa_prefill_causal_ws": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _P, _SZ, _P]),
    "sa_prefill_causal_strided_ws": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _F, _P, _P, _SZ,
                                          _P]),
    "sa_set_attention_blocks": (_I, [_I, _I]),
    "sa_get_attention_blocks": (_I, [C.POINTER(_I), C.POINTER(_I)]),
    "sa_prefill_query_tile": (_I, [_I, _I, _I, _I, _I, _I]),
    "sa_qwen3_create": (_I, [C.POINTER(Qwen3Desc), _I, C.POINTER(_P)]),
    "sa_qwen3_destroy": (_I, [_P]),
    "sa_qwen3_get_desc": (_I, [_P, C.POINTER(Qwen3Desc)]),
    "sa_qwen3_tensor_ptr": (_I, [_P, _I, _I, C.POINTER(_P), C.POINTER(_SZ), C.POINTER(_I)]),
    "sa_qwen3_desc_from_safetensors": (_I, [C.c_char_p, C.POINTER(Qwen3Desc)]),
    "sa_qwen3_load_safetensors": (_I, [_P, C.c_char_p]),
    "sa_qwen3_init_random": (_I, [_P, C.c_uint64, _F, _P]),
    "sa_qwen3_decode_step": (_I, [_P, _P, _P, _I, _P, _P, _P]),
    "sa_qwen3_prefill": (_I, [_P, _P, _P, _I, _I, _P, _P, _P]),
}

_lib = None


def lib() -> C.CDLL:
    """Load libsa_amd.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run `python streaming-attention_amd/build.py`")
        # RTLD_LOCAL: the library exports the reference API's C++ names, which
        # must not interpose on another library loaded into the same process.
        handle = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != SA_OK:
        raise SaError(status, lib().sa_last_error().decode())


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _rows(ids, n: int):
    """Host int32 array of cache rows for the C ABI (None stays NULL)."""
    if ids is None:
        return None
    ids = [int(i) for i in ids]
    if len(ids) != n:
        raise ValueError(f"seq_ids has {len(ids)} entries for {n} sequences")
    return C.cast((C.c_int32 * n)(*ids), C.c_void_p)


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else stream


def _f32(t, name: str):
    import torch
    if t is None:
        return None
    if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 CUDA tensor")
    return t


# ---------------------------------------------------------------- single query

def stream_attn(Q, K, V, block_size: int = 64, scale: float = 1.0, out=None, ws=None, stream=None):
    """O = softmax(scale Q K^T) V for Q [d], K/V [T, d] (fp32, device)."""
    import torch
    T, d = (K.shape[0], K.shape[1]) if K.dim() == 2 else (0, Q.numel())
    out = torch.empty(d, dtype=torch.float32, device=Q.device) if out is None else out
    need = lib().sa_stream_attn_ws_bytes(T, d)
    if ws is None and need:
        ws = torch.zeros(need, dtype=torch.uint8, device=Q.device)
    check(lib().sa_stream_attn_f32(_ptr(_f32(Q, "Q")), _ptr(_f32(K, "K")), _ptr(_f32(V, "V")), T, d,
                                   block_size, scale, _ptr(out), _ptr(ws), 0 if ws is None else ws.numel(),
                                   _stream(stream)))
    return out


def decode_dense(q, k, v, scale: float, out=None, ws=None, stream=None):
    """q [B, Hq, D], k/v [B, Hkv, T, D] -> out [B, Hq, D] (fp32)."""
    import torch
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    out = torch.empty_like(q) if out is None else out
    need = lib().sa_decode_dense_ws_bytes(B, Hq, T, D)
    if ws is None and need:
        ws = torch.zeros(need, dtype=torch.uint8, device=q.device)
    check(lib().sa_decode_dense_f32(_ptr(_f32(q, "q")), _ptr(_f32(k, "k")), _ptr(_f32(v, "v")), B, Hq,
                                    Hkv, T, D, scale, _ptr(out), _ptr(ws),
                                    0 if ws is None else ws.numel(), _stream(stream)))
    return out


# ---------------------------------------------------------------- KV cache

class KVCache:
    """Owner of an sa_kvcache handle (64-token pages, fp32 or bf16 storage)."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, max_seqs: int,
                 max_pages_per_seq: int, num_pages: int, kv_dtype: int = SA_DTYPE_F32):
        self.desc = KvDesc(num_layers, num_kv_heads, head_dim, max_seqs, max_pages_per_seq,
                           num_pages, kv_dtype)
        h = C.c_void_p()
        check(lib().sa_kvcache_create(C.byref(self.desc), C.byref(h)))
        self.handle = h

    def close(self) -> None:
        if self.handle:
            lib().sa_kvcache_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self, stream=None) -> None:
        check(lib().sa_kvcache_reset(self.handle, _stream(stream)))

    def reserve(self, seq: int, n_tokens: int, stream=None) -> None:
        check(lib().sa_kvcache_reserve(self.handle, seq, n_tokens, _stream(stream)))

    def set_pages(self, seq: int, pages, stream=None) -> None:
        arr = (C.c_int32 * max(len(pages), 1))(*[int(p) for p in pages])
        check(lib().sa_kvcache_set_pages(self.handle, seq, arr, len(pages), _stream(stream)))

    def set_len(self, seq: int, n: int, stream=None) -> None:
        check(lib().sa_kvcache_set_len(self.handle, seq, n, _stream(stream)))

    def length(self, seq: int) -> int:
        return lib().sa_kvcache_len(self.handle, seq)

    def capacity(self, seq: int) -> int:
        """Tokens the pages assigned to seq can hold, or -1."""
        return lib().sa_kvcache_capacity(self.handle, seq)

    def commit(self, n: int, seqs=None, n_seqs: int | None = None, stream=None) -> None:
        if seqs is None:
            check(lib().sa_kvcache_commit(self.handle, None, n_seqs or 0, n, _stream(stream)))
        else:
            arr = (C.c_int32 * len(seqs))(*[int(s) for s in seqs])
            check(lib().sa_kvcache_commit(self.handle, arr, len(seqs), n, _stream(stream)))

    def k_pool(self, layer: int) -> int:
        return lib().sa_kvcache_k_pool(self.handle, layer)

    def v_pool(self, layer: int) -> int:
        return lib().sa_kvcache_v_pool(self.handle, layer)

    def nbytes(self) -> int:
        return lib().sa_kvcache_bytes(self.handle)

    def append(self, layer: int, q, k, v, q_norm_w=None, k_norm_w=None, eps: float = 1e-6,
               rope=None, q_out=None, seq_ids=None, stream=None):
        """q [n, S, Hq, D] (or None), k/v [n, S, Hkv, D]; rope = (cos, sin) tables;
        seq_ids: cache rows of the n sequences (host ints), or None for 0..n-1."""
        n_seq, S = k.shape[0], k.shape[1]
        Hq = 0 if q is None else q.shape[2]
        cos, sin = (None, None) if rope is None else rope
        max_pos = 0 if rope is None else cos.shape[0]
        if q is not None and q_out is None:
            import torch
            q_out = torch.empty_like(q)
        check(lib().sa_qknorm_rope_append(
            self.handle, layer, _ptr(_f32(q, "q")), _ptr(_f32(k, "k")), _ptr(_f32(v, "v")), n_seq, S,
            _rows(seq_ids, n_seq), Hq, _ptr(_f32(q_norm_w, "q_norm_w")), _ptr(_f32(k_norm_w, "k_norm_w")), eps,
            _ptr(cos), _ptr(sin), max_pos, _ptr(q_out), _stream(stream)))
        return q_out

    def decode_ws_bytes(self, n_seq: int, n_q_heads: int) -> int:
        return lib().sa_paged_decode_ws_bytes(self.handle, n_seq, n_q_heads)

    def decode(self, layer: int, q, scale: float, n_pending: int = 0, out=None, ws=None,
               seq_ids=None, stream=None):
        """q [n_seq, Hq, D] -> out [n_seq, Hq, D]; seq_ids: cache rows (host
        ints) or None for 0..n_seq-1."""
        import torch
        n_seq, Hq, _ = q.shape
        out = torch.empty_like(q) if out is None else out
        if ws is None:
            need = self.decode_ws_bytes(n_seq, Hq)
            ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=q.device)
        check(lib().sa_paged_decode(self.handle, layer, _ptr(_f32(q, "q")), n_seq, _rows(seq_ids, n_seq), Hq,
                                    n_pending, scale, _ptr(out), _ptr(ws), ws.numel(), _stream(stream)))
        return out

    def append_decode(self, layer: int, q, k, v, scale: float, q_norm_w=None, k_norm_w=None, eps: float = 1e-6,
                      rope=None, out=None, q_out=None, ws=None, commit: bool = False, seq_ids=None, stream=None):
        """One decode step in one call: q [n_seq, Hq, D] and k/v [n_seq, Hkv, D]
        of the new token (before norm and RoPE) -> out [n_seq, Hq, D], the
        attention over the cache plus the token; commit=True also commits it.
        q_out, if given, receives the normed, rotated q."""
        import torch
        n_seq, Hq, _ = q.shape
        out = torch.empty_like(q) if out is None else out
        if ws is None:
            need = self.decode_ws_bytes(n_seq, Hq)
            ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=q.device)
        cos, sin = (None, None) if rope is None else rope
        max_pos = 0 if rope is None else cos.shape[0]
        check(lib().sa_append_decode(
            self.handle, layer, _ptr(_f32(q, "q")), _ptr(_f32(k, "k")), _ptr(_f32(v, "v")), n_seq,
            _rows(seq_ids, n_seq), Hq, _ptr(_f32(q_norm_w, "q_norm_w")), _ptr(_f32(k_norm_w, "k_norm_w")), eps,
            _ptr(cos), _ptr(sin), max_pos, scale, _ptr(out), _ptr(q_out), _ptr(ws), ws.numel(), int(bool(commit)),
            _stream(stream)))
        return out

    def append_decode_partials(self, layer: int, part, n_q_heads: int, scale: float, q_norm_w=None,
                               k_norm_w=None, eps: float = 1e-6, rope=None, out=None, q_out=None, ws=None,
                               commit: bool = False, seq_ids=None, stream=None):
        """append_decode with q, k and v of the new token given as split-K
        partials: part [n_part, n_seq, (Hq + 2 Hkv) D], summed in order."""
        import torch
        n_part, n_seq, _ = part.shape
        D = self.desc.head_dim
        out = torch.empty(n_seq, n_q_heads, D, dtype=torch.float32, device=part.device) if out is None else out
        if ws is None:
            need = self.decode_ws_bytes(n_seq, n_q_heads)
            ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=part.device)
        cos, sin = (None, None) if rope is None else rope
        max_pos = 0 if rope is None else cos.shape[0]
        check(lib().sa_append_decode_partials(
            self.handle, layer, _ptr(_f32(part, "part")), n_part, n_seq, _rows(seq_ids, n_seq), n_q_heads,
            _ptr(_f32(q_norm_w, "q_norm_w")), _ptr(_f32(k_norm_w, "k_norm_w")), eps, _ptr(cos), _ptr(sin), max_pos,
            scale, _ptr(out), _ptr(q_out), _ptr(ws), ws.numel(), int(bool(commit)), _stream(stream)))
        return out

    def gather(self, layer: int, seq: int, length: int, stream=None):
        import torch
        H, D = self.desc.num_kv_heads, self.desc.head_dim
        k = torch.empty(H, length, D, dtype=torch.float32, device="cuda")
        v = torch.empty_like(k)
        check(lib().sa_kvcache_gather(self.handle, layer, seq, length, _ptr(k), _ptr(v),
                                      _stream(stream)))
        return k, v


def rope_tables(max_pos: int, head_dim: int, theta: float = 1e6, device="cuda"):
    import torch
    cos = torch.empty(max_pos, head_dim // 2, dtype=torch.float32, device=device)
    sin = torch.empty_like(cos)
    check(lib().sa_rope_table_init(_ptr(cos), _ptr(sin), max_pos, head_dim, theta, _stream(None)))
    return cos, sin


SA_NORM_EPS_INSIDE, SA_NORM_EPS_OUTSIDE = 0, 1


def qk_norm_rope(x, pos, norm_w=None, eps: float = 1e-6, rope=None, out=None, stream=None,
                 eps_outside: bool = False):
    """Per-row RMSNorm (weights norm_w [D], or none) and rotate-half RoPE (rope =
    (cos, sin) tables, or none) of x [..., D] fp32 at positions pos (int32
    [rows]); out may alias x.  eps_outside: x / (sqrt(mean(x^2)) + eps)."""
    import torch
    D = x.shape[-1]
    rows = x.numel() // D
    if pos.dtype != torch.int32 or pos.numel() != rows:
        raise ValueError("pos must be int32 with one entry per row")
    out = torch.empty_like(x) if out is None else out
    cos, sin = rope if rope is not None else (None, None)
    mode = SA_NORM_EPS_OUTSIDE if eps_outside else SA_NORM_EPS_INSIDE
    check(lib().sa_qk_norm_rope_ex(_ptr(_f32(x, "x")), rows, D, _ptr(pos), _ptr(norm_w), eps, mode, _ptr(cos),
                                   _ptr(sin), cos.shape[0] if cos is not None else 0, _ptr(out),
                                   _stream(stream)))
    return out


# ---------------------------------------------------------------- dense fp32 operators

def linear(x, w, bias=None, out=None, stream=None):
    """x [..., K] . w[N][K]^T (+ bias [N]) -> [..., N], fp32 (ops::linear)."""
    import torch
    K = x.shape[-1]
    if w.dim() != 2 or w.shape[1] != K:
        raise ValueError("w must be [N, K] with K = x.shape[-1]")
    N = w.shape[0]
    M = 1
    for n in x.shape[:-1]:
        M *= n
    out = torch.empty(*x.shape[:-1], N, dtype=torch.float32, device=x.device) if out is None else out
    check(lib().sa_linear_f32(_ptr(_f32(x, "x")), M, K, _ptr(_f32(w, "w")), N,
                              _ptr(_f32(bias, "bias")) if bias is not None else None, _ptr(out),
                              _stream(stream)))
    return out


def rms_norm(x, w=None, eps: float = 1e-6, out=None, stream=None):
    """x / sqrt(mean(x^2) + eps) * w over the last axis (ops::rms_norm)."""
    import torch
    n = x.shape[-1]
    out = torch.empty_like(x) if out is None else out
    check(lib().sa_rms_norm_f32(_ptr(_f32(x, "x")), x.numel() // n, n,
                                _ptr(_f32(w, "w")) if w is not None else None, eps, _ptr(out), _stream(stream)))
    return out


def swiglu(gate, up, out=None, stream=None):
    """up * silu(gate), elementwise (qwen3_mlp's activation)."""
    import torch
    if gate.shape != up.shape:
        raise ValueError("gate and up must have one shape")
    out = torch.empty_like(gate) if out is None else out
    check(lib().sa_swiglu_f32(_ptr(_f32(gate, "gate")), _ptr(_f32(up, "up")), gate.numel(), _ptr(out),
                              _stream(stream)))
    return out


def axpby(x, a: float, y=None, b: float = 0.0, out=None, stream=None):
    """a x + b y (or a x without y), elementwise."""
    import torch
    if y is not None and y.shape != x.shape:
        raise ValueError("x and y must have one shape")
    out = torch.empty_like(x) if out is None else out
    check(lib().sa_axpby_f32(_ptr(_f32(x, "x")), a, _ptr(_f32(y, "y")) if y is not None else None, b,
                             x.numel(), _ptr(out), _stream(stream)))
    return out


# ---------------------------------------------------------------- prefill

def set_attention_blocks(q_block: int = 0, kv_block: int = 0) -> None:
    """Process-wide attention tiles (0 = the launch's own choice): prefill
    query rows per workgroup and head, decode split-KV chunk tokens."""
    check(lib().sa_set_attention_blocks(int(q_block), int(kv_block)))


def get_attention_blocks() -> tuple[int, int]:
    q, kv = C.c_int(), C.c_int()
    check(lib().sa_get_attention_blocks(C.byref(q), C.byref(kv)))
    return q.value, kv.value


def prefill_query_tile(dtype: int, batch: int, n_q_heads: int, n_kv_heads: int, L: int, D: int) -> int:
    """Query rows per workgroup and head of a prefill launch of this shape."""
    r = lib().sa_prefill_query_tile(dtype, batch, n_q_heads, n_kv_heads, L, D)
    if r < 0:
        check(r)
    return r


def prefill_ws_bytes(dtype: int, batch: int, n_q_heads: int, n_kv_heads: int, L: int, D: int) -> int:
    """Workspace bytes of a prefill launch of this shape (0: it takes none)."""
    return int(lib().sa_prefill_causal_ws_bytes(dtype, batch, n_q_heads, n_kv_heads, L, D))


def prefill_causal(q, k, v, scale: float, out=None, stream=None, ws=None):
    """q [B, Hq, L, D], k/v [B, Hkv, L, D] (fp32 or bf16) -> out fp32 [B, Hq, L, D].
    ws: a CUDA tensor of at least prefill_ws_bytes bytes (sa_prefill_causal_ws),
    or None (sa_prefill_causal)."""
    import torch
    if q.dtype == torch.float32:
        dt = SA_DTYPE_F32
    elif q.dtype == torch.bfloat16:
        dt = SA_DTYPE_BF16
    else:
        raise ValueError("q must be float32 or bfloat16")
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        if t.dtype != q.dtype or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{n} must be a contiguous CUDA tensor of q's dtype")
    B, Hq, L, D = q.shape
    Hkv = k.shape[1]
    out = torch.empty(B, Hq, L, D, dtype=torch.float32, device=q.device) if out is None else out
    if ws is None:
        check(lib().sa_prefill_causal(_ptr(q), _ptr(k), _ptr(v), dt, B, Hq, Hkv, L, D, scale, _ptr(out),
                                      _stream(stream)))
    else:
        check(lib().sa_prefill_causal_ws(_ptr(q), _ptr(k), _ptr(v), dt, B, Hq, Hkv, L, D, scale, _ptr(out),
                                         _ptr(ws), ws.numel() * ws.element_size(), _stream(stream)))
    return out


# ---------------------------------------------------------------- Qwen3 decoder

QW_EMBED, QW_IN_NORM, QW_QKV, QW_Q_NORM, QW_K_NORM, QW_O, QW_POST_NORM, QW_GATE_UP, QW_DOWN, \
    QW_FINAL_NORM, QW_LM_HEAD = range(11)
QW_GLOBAL = (QW_EMBED, QW_FINAL_NORM, QW_LM_HEAD)

QWEN3_0_6B = dict(num_layers=28, hidden=1024, intermediate=3072, vocab=151936, n_q_heads=16,
                  n_kv_heads=8, head_dim=128, rms_eps=1e-6, rope_theta=1e6)


class Qwen3:
    """Owner of an sa_qwen3 handle: bf16 weights on the device and the greedy
    decode step of include/sa_qwen3.h."""

    def __init__(self, max_batch: int, max_pos: int, **shape):
        d = dict(QWEN3_0_6B)
        d.update(shape)
        self.desc = Qwen3Desc(d["num_layers"], d["hidden"], d["intermediate"], d["vocab"],
                              d["n_q_heads"], d["n_kv_heads"], d["head_dim"], max_pos, d["rms_eps"],
                              d["rope_theta"])
        h = C.c_void_p()
        check(lib().sa_qwen3_create(C.byref(self.desc), max_batch, C.byref(h)))
        self.handle = h
        self.max_batch = max_batch

    @staticmethod
    def checkpoint_shape(path) -> dict:
        """The model shape a safetensors checkpoint holds (host only)."""
        d = Qwen3Desc()
        check(lib().sa_qwen3_desc_from_safetensors(os.fsencode(path), C.byref(d)))
        return {f: getattr(d, f) for f, _ in Qwen3Desc._fields_ if f != "max_pos"}

    @classmethod
    def from_safetensors(cls, path, max_batch: int, max_pos: int) -> "Qwen3":
        """A model of the checkpoint's shape with its weights uploaded."""
        m = cls(max_batch, max_pos, **cls.checkpoint_shape(path))
        m.load_safetensors(path)
        return m

    def load_safetensors(self, path) -> None:
        """Upload a checkpoint of this model's shape (synchronous)."""
        check(lib().sa_qwen3_load_safetensors(self.handle, os.fsencode(path)))

    def close(self) -> None:
        if self.handle:
            lib().sa_qwen3_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor_ptr(self, which: int, layer: int = 0):
        """(device pointer, element count, dtype code) of one weight tensor."""
        p, n, dt = C.c_void_p(), C.c_size_t(), C.c_int()
        check(lib().sa_qwen3_tensor_ptr(self.handle, layer, which, C.byref(p), C.byref(n), C.byref(dt)))
        return p.value, n.value, dt.value

    def tensor(self, which: int, layer: int = 0):
        """A torch view of one weight tensor (bfloat16 or float32, flat)."""
        import torch
        ptr, n, dt = self.tensor_ptr(which, layer)
        return _device_view(ptr, n, torch.bfloat16 if dt == SA_DTYPE_BF16 else torch.float32)

    def init_random(self, seed: int, std: float = 0.02, stream=None) -> None:
        check(lib().sa_qwen3_init_random(self.handle, seed, std, _stream(stream)))

    def prefill(self, cache: "KVCache", tokens, next_tokens=None, logits=None, stream=None):
        """tokens: int32 CUDA [B][L] prompts of empty sequences 0..B-1 -> next
        tokens int32 CUDA [B] (and the last position's logits if given)."""
        import torch
        if tokens.dtype != torch.int32 or not tokens.is_cuda or tokens.dim() != 2:
            raise ValueError("tokens must be an int32 CUDA tensor [B][L]")
        tokens = tokens.contiguous()
        B, L = tokens.shape
        next_tokens = torch.empty(B, dtype=torch.int32, device=tokens.device) if next_tokens is None else next_tokens
        check(lib().sa_qwen3_prefill(self.handle, cache.handle, _ptr(tokens), B, L, _ptr(next_tokens), _ptr(logits),
                                     _stream(stream)))
        return next_tokens

    def decode_step(self, cache: "KVCache", tokens, next_tokens=None, logits=None, stream=None):
        """tokens: int32 CUDA [B] -> next tokens int32 CUDA [B] (and logits if given)."""
        import torch
        B = tokens.shape[0]
        if tokens.dtype != torch.int32 or not tokens.is_cuda:
            raise ValueError("tokens must be an int32 CUDA tensor")
        next_tokens = torch.empty_like(tokens) if next_tokens is None else next_tokens
        check(lib().sa_qwen3_decode_step(self.handle, cache.handle, _ptr(tokens), B, _ptr(next_tokens),
                                         _ptr(logits), _stream(stream)))
        return next_tokens


class _CudaArray:
    """__cuda_array_interface__ over memory this library owns (no copy)."""

    def __init__(self, ptr: int, n: int, typestr: str):
        self.__cuda_array_interface__ = {"shape": (n,), "typestr": typestr, "data": (ptr, False),
                                         "version": 2, "strides": None}


def _device_view(ptr: int, n: int, dtype):
    import torch
    if dtype == torch.bfloat16:
        # torch has no bfloat16 typestr: view the bits as int16
        return torch.as_tensor(_CudaArray(ptr, n, "<i2"), device="cuda").view(torch.bfloat16)
    return torch.as_tensor(_CudaArray(ptr, n, "<f4"), device="cuda")


def kv_pool_views(cache: "KVCache", layer: int):
    """Flat torch views of one layer's K and V page pools (storage dtype)."""
    import torch
    d = cache.desc
    n = d.num_pages * d.num_kv_heads * PAGE_TOKENS * d.head_dim
    dt = torch.bfloat16 if d.kv_dtype == SA_DTYPE_BF16 else torch.float32
    return _device_view(cache.k_pool(layer), n, dt), _device_view(cache.v_pool(layer), n, dt)
