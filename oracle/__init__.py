"""CPU oracle for the ytensor_amd hot path — TEST INFRASTRUCTURE ONLY.

Two libraries share one C ABI shape:

* ``liboracle.so`` — the from-scratch restatement in ``ytoracle.cpp`` of
  YTensor's CPU algorithms (SnifferCaptain/ytensor v0.13). Always built.
* ``_ref/libytref.so`` — the reference itself compiled from its own sources
  by ``make ref`` (only where ``/root/reference`` exists). Optional.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker / the timed CPU baseline.
The product path (``ytensor_amd``) never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libytref.so")
REF_ROOT = "/root/reference"

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float


def build(ref: bool | None = None) -> None:
    """Compile liboracle.so (and _ref/libytref.so when the reference exists)."""
    subprocess.check_call(["make", "-s", "-C", HERE, "all"])
    if ref is None:
        ref = os.path.isdir(REF_ROOT)
    if ref:
        subprocess.check_call(["make", "-s", "-C", HERE, "ref"])


def _bind(lib: ctypes.CDLL, prefix: str) -> ctypes.CDLL:
    sig = {
        "seed": (None, [ctypes.c_uint32]),
        "randn": (None, [_P, _L]),
        "bf16_round": (None, [_P, _P, _L]),
        "bf16_to_f32": (None, [_P, _P, _L]),
        "f16_round": (None, [_P, _P, _L]),
        "f16_to_f32": (None, [_P, _P, _L]),
        "sgemm": (None, [_P, _P, _P, _I, _I, _I, _F, _F, _L, _L, _L, _L, _L, _L]),
        "flash_attention": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _F] + [_L] * 8 + [_P, _L, _P, _L, _L]),
        "sdpa_gqa": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I]),
        "rms_norm": (None, [_P, _P, _L, _I, _F]),
        "rope_precompute": (None, [_I, _I, _F, _P, _P]),
        "rope": (None, [_P, _I, _I, _I, _I, _P, _P]),
        "qwen3_generate": (_I, [_P, _P, _P, _P, _I, _I, _P, _P, _P]),
        "qwen3_run": (_I, [_P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P]),
        "sgemm_masked": (None, [_P, _P, _P, _I, _I, _I, _F, _F, _L, _L, _L, _L, _L, _L, _P]),
        "sdpa_math": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _I, _I]),
        "sdpa_ex": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _I, _I, _I]),
        "masked_matmul": (None, [_P, _P, _P, _I, _I, _I, _P, _I, _I, _F]),
        "yt_save": (_I, [ctypes.c_char_p, _I, _P, _P, _P, _P, _P, ctypes.c_char_p, _I]),
        "yt_names": (_I, [ctypes.c_char_p, _P, _L]),
        "yt_load": (_I, [ctypes.c_char_p, ctypes.c_char_p, _P, _L, _P, _P, _I, _P, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, f"{prefix}_{name}", None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    return lib


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


class CpuPath:
    """numpy-facing wrapper over one of the two libraries."""

    def __init__(self, path: str, prefix: str):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run `make -C {HERE}`)")
        self.lib = _bind(ctypes.CDLL(path), prefix)
        self.prefix = prefix
        self.path = path

    def _fn(self, name):
        return getattr(self.lib, f"{self.prefix}_{name}")

    # --- RNG (YTensor::seed / YTensor::randn) ---------------------------------
    def seed(self, s: int) -> None:
        self._fn("seed")(s)

    def randn(self, *shape: int) -> np.ndarray:
        out = np.empty(shape, dtype=np.float32)
        self._fn("randn")(_ptr(out), out.size)
        return out

    # --- type conversions ------------------------------------------------------
    def bf16_round(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=np.uint16)
        self._fn("bf16_round")(_ptr(x), _ptr(out), x.size)
        return out

    def bf16_to_f32(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, dtype=np.float32)
        self._fn("bf16_to_f32")(_ptr(h), _ptr(out), h.size)
        return out

    def f16_round(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=np.uint16)
        self._fn("f16_round")(_ptr(x), _ptr(out), x.size)
        return out

    def f16_to_f32(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, dtype=np.float32)
        self._fn("f16_to_f32")(_ptr(h), _ptr(out), h.size)
        return out

    # --- GEMM ------------------------------------------------------------------
    def sgemm(self, A: np.ndarray, B: np.ndarray, *, b_trans: bool = False, alpha: float = 1.0,
              beta: float = 0.0, C: np.ndarray | None = None) -> np.ndarray:
        """C = alpha*A@B + beta*C. A [m,k] row-major; B [k,n] row-major, or
        (b_trans) W [n,k] row-major passed as the column-major view B = W^T."""
        A = np.ascontiguousarray(A, dtype=np.float32)
        B = np.ascontiguousarray(B, dtype=np.float32)
        m, k = A.shape
        if b_trans:
            n = B.shape[0]
            rsb, csb = 1, k
        else:
            n = B.shape[1]
            rsb, csb = n, 1
        if C is None:
            C = np.zeros((m, n), dtype=np.float32)
        else:
            C = np.ascontiguousarray(C, dtype=np.float32).copy()
        self._fn("sgemm")(_ptr(A), _ptr(B), _ptr(C), m, n, k, alpha, beta, k, 1, rsb, csb, n, 1)
        return C

    # --- attention ---------------------------------------------------------------
    def flash_attention(self, Q, K, V, scale, mask=None, bias=None) -> np.ndarray:
        """One matrix: Q [q,d], K [kv,d], V [kv,dv] contiguous; mask bool [q,kv]."""
        Q = np.ascontiguousarray(Q, dtype=np.float32)
        K = np.ascontiguousarray(K, dtype=np.float32)
        V = np.ascontiguousarray(V, dtype=np.float32)
        q_len, d = Q.shape
        kv_len, dv = V.shape
        O = np.zeros((q_len, dv), dtype=np.float32)
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self._fn("flash_attention")(
            _ptr(Q), _ptr(K), _ptr(V), _ptr(O), q_len, kv_len, d, dv, scale,
            d, 1, d, 1, dv, 1, dv, 1,
            _ptr(m), kv_len, _ptr(b), kv_len if b is not None else 0, 1)
        return O

    def sdpa_gqa(self, Q, K, V, scale=0.0, causal=True) -> np.ndarray:
        """Q [B,Hq,S,D], K/V [B,Hkv,KV,D] contiguous float32 -> O [B,Hq,S,D]."""
        Q = np.ascontiguousarray(Q, dtype=np.float32)
        K = np.ascontiguousarray(K, dtype=np.float32)
        V = np.ascontiguousarray(V, dtype=np.float32)
        B, Hq, S, D = Q.shape
        Hkv, KV = K.shape[1], K.shape[2]
        O = np.zeros_like(Q)
        self._fn("sdpa_gqa")(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), B, Hq, Hkv, S, KV, D, scale, int(causal))
        return O

    # --- masked matmul / MATH SDPA -----------------------------------------------
    def sgemm_masked(self, A, B, C, mask, alpha=1.0, beta=0.0):
        """sgemm_masked on contiguous A [m,k], B [k,n]; C [m,n] updated in place
        where mask [m,n] is set (returned)."""
        A = np.ascontiguousarray(A, dtype=np.float32)
        B = np.ascontiguousarray(B, dtype=np.float32)
        assert C.flags.c_contiguous and C.dtype == np.float32
        mk = np.ascontiguousarray(mask, dtype=np.uint8)
        m, k = A.shape
        n = B.shape[1]
        self._fn("sgemm_masked")(_ptr(A), _ptr(B), _ptr(C), m, n, k, alpha, beta, k, 1, n, 1, n, 1, _ptr(mk))
        return C

    def sdpa_math(self, Q, K, V, scale=0.0, mask=None, bias=None, diag=None):
        """scaledDotProductAttention(MATH) over [H, L, D] fp32 tensors; mask bool
        [Lq, Lkv], or diag = offset for the predicate j <= i + offset."""
        return self._sdpa(Q, K, V, scale, mask, bias, diag, 0)

    def sdpa_flash(self, Q, K, V, scale=0.0, mask=None, bias=None, diag=None):
        """scaledDotProductAttention(FLASH_AVX2) through the tensor API (reference only)."""
        return self._sdpa(Q, K, V, scale, mask, bias, diag, 1)

    def _sdpa(self, Q, K, V, scale, mask, bias, diag, backend):
        Q = np.ascontiguousarray(Q, dtype=np.float32)
        K = np.ascontiguousarray(K, dtype=np.float32)
        V = np.ascontiguousarray(V, dtype=np.float32)
        H, Lq, D = Q.shape
        Lkv, Dv = V.shape[1], V.shape[2]
        O = np.zeros((H, Lq, Dv), np.float32)
        mk = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
        bs = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        dg, off = (0, 0) if diag is None else (1, int(diag))
        if self.prefix == "ref":
            self._fn("sdpa_ex")(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), H, Lq, Lkv, D, Dv, scale, _ptr(mk), _ptr(bs),
                                backend, dg, off)
        else:
            if backend != 0:
                raise NotImplementedError("the oracle's FLASH is flash_attention / sdpa_gqa")
            self._fn("sdpa_math")(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), H, Lq, Lkv, D, Dv, scale, _ptr(mk), _ptr(bs),
                                  dg, off)
        return O

    def masked_matmul(self, A, B, mask=None, diag=None, value=0.0):
        """YTensor::masked_matmul (reference) / fill + sgemm_masked (oracle)."""
        A = np.ascontiguousarray(A, dtype=np.float32)
        B = np.ascontiguousarray(B, dtype=np.float32)
        m, k = A.shape
        n = B.shape[1]
        if self.prefix == "ref":
            O = np.empty((m, n), np.float32)
            mk = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
            dg, off = (0, 0) if diag is None else (1, int(diag))
            self._fn("masked_matmul")(_ptr(A), _ptr(B), _ptr(O), m, n, k, _ptr(mk), dg, off, value)
            return O
        if diag is not None:
            mask = np.arange(n)[None, :] <= np.arange(m)[:, None] + int(diag)
        O = np.full((m, n), value, np.float32)
        return self.sgemm_masked(A, B, O, mask)

    # --- RMSNorm / RoPE ----------------------------------------------------------
    def rms_norm(self, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        w = np.ascontiguousarray(w, dtype=np.float32)
        n = x.shape[-1]
        self._fn("rms_norm")(_ptr(x), _ptr(w), x.size // n, n, eps)
        return x

    def rope_tables(self, dim: int, max_len: int, theta: float):
        c = np.empty((max_len, dim), dtype=np.float32)
        s = np.empty((max_len, dim), dtype=np.float32)
        self._fn("rope_precompute")(dim, max_len, theta, _ptr(c), _ptr(s))
        return c, s

    def rope(self, x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
        """x [B,H,L,D]; cos/sin [L,D] (already sliced to the positions)."""
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        B, H, L, D = x.shape
        cos = np.ascontiguousarray(cos[:L], dtype=np.float32)
        sin = np.ascontiguousarray(sin[:L], dtype=np.float32)
        self._fn("rope")(_ptr(x), B, H, L, D, _ptr(cos), _ptr(sin))
        return x

    def qwen3_generate(self, cfg: "Qwen3Config", weights: np.ndarray, prompt, n_steps: int):
        """Greedy generation with the Qwen3 decoder (flat fp32 weight buffer in
        qwen3_weight_layout order). Returns (tokens, top1-top2 margins, first-step logits)."""
        ci = np.array([cfg.hidden, cfg.layers, cfg.vocab, cfg.inter, cfg.n_heads, cfg.n_kv, cfg.head_dim,
                       cfg.max_pos], dtype=np.int32)
        cf = np.array([cfg.eps, cfg.theta], dtype=np.float32)
        w = np.ascontiguousarray(weights, dtype=np.float32)
        pr = np.ascontiguousarray(prompt, dtype=np.int32)
        toks = np.zeros(n_steps, np.int32)
        marg = np.zeros(n_steps, np.float32)
        lg0 = np.zeros(cfg.vocab, np.float32)
        st = self._fn("qwen3_generate")(_ptr(ci), _ptr(cf), _ptr(w), _ptr(pr), len(pr), n_steps, _ptr(toks),
                                        _ptr(marg), _ptr(lg0))
        if st != 0:
            raise ValueError(f"qwen3_generate failed ({st})")
        return toks, marg, lg0

    def qwen3_run(self, cfg: "Qwen3Config", weights: np.ndarray, turns, logit_steps=()):
        """Greedy multi-turn generation over one set of KV caches (the caches
        wrap once more than cfg.max_pos tokens were written). turns: list of
        (prompt tokens, n_steps). Returns (tokens, margins, logits [len(logit_steps), V])
        with one token / margin per step of all turns in order."""
        ci = np.array([cfg.hidden, cfg.layers, cfg.vocab, cfg.inter, cfg.n_heads, cfg.n_kv, cfg.head_dim,
                       cfg.max_pos], dtype=np.int32)
        cf = np.array([cfg.eps, cfg.theta], dtype=np.float32)
        w = np.ascontiguousarray(weights, dtype=np.float32)
        lens = np.array([len(p) for p, _ in turns], np.int32)
        steps = np.array([n for _, n in turns], np.int32)
        prompts = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int32) for p, _ in turns]))
        total = int(steps.sum())
        toks = np.zeros(total, np.int32)
        marg = np.zeros(total, np.float32)
        ls = np.ascontiguousarray(np.asarray(logit_steps, np.int32).reshape(-1))
        lg = np.zeros((max(len(ls), 1), cfg.vocab), np.float32)
        st = self._fn("qwen3_run")(_ptr(ci), _ptr(cf), _ptr(w), len(turns), _ptr(lens), _ptr(prompts), _ptr(steps),
                                   _ptr(toks), _ptr(marg), _ptr(ls) if len(ls) else None, len(ls), _ptr(lg))
        if st != 0:
            raise ValueError(f"qwen3_run failed ({st})")
        return toks, marg, lg[:len(ls)]

    # --- .yt files (the compiled reference's yt::io::YTensorIO only) ----------
    def yt_save(self, path: str, tensors, compress: str = "", mode: int = 2) -> None:
        """tensors: [(name, typeName, shape, numpy payload)]; mode 2 = Write, 3 = Append."""
        n = len(tensors)
        names = (ctypes.c_char_p * max(1, n))(*[t[0].encode() for t in tensors])
        dts = (ctypes.c_char_p * max(1, n))(*[t[1].encode() for t in tensors])
        nd = (ctypes.c_int * max(1, n))(*[len(t[2]) for t in tensors])
        dims = [int(d) for t in tensors for d in t[2]]
        sh = (ctypes.c_int * max(1, len(dims)))(*dims)
        arrs = [np.ascontiguousarray(t[3]) for t in tensors]
        ptrs = (ctypes.c_void_p * max(1, n))(*[a.ctypes.data for a in arrs])
        st = self._fn("yt_save")(path.encode(), n, ctypes.cast(names, _P), ctypes.cast(dts, _P),
                                 ctypes.cast(nd, _P), ctypes.cast(sh, _P), ctypes.cast(ptrs, _P),
                                 compress.encode(), mode)
        if st != 0:
            raise ValueError(f"reference save failed ({st})")

    def yt_names(self, path: str) -> list[str]:
        buf = ctypes.create_string_buffer(1 << 16)
        n = self._fn("yt_names")(path.encode(), ctypes.cast(buf, _P), len(buf))
        if n < 0:
            raise ValueError("reference open failed")
        return buf.value.decode().split("\n")[:n]

    def yt_load(self, path: str, name: str = "", cap: int = 1 << 26):
        """-> (typeName, shape, bytes) as YTensorIO::load returns them."""
        out = np.empty(cap, np.uint8)
        nb = ctypes.c_int64()
        dt = ctypes.create_string_buffer(64)
        nd = ctypes.c_int()
        shape = (ctypes.c_int * 16)()
        st = self._fn("yt_load")(path.encode(), name.encode(), _ptr(out), cap, ctypes.byref(nb),
                                 ctypes.cast(dt, _P), 64, ctypes.byref(nd), ctypes.cast(shape, _P))
        if st != 0:
            raise ValueError(f"reference load failed ({st})")
        return dt.value.decode(), [shape[i] for i in range(nd.value)], out[:nb.value].tobytes()

    def set_num_threads(self, t: int) -> None:
        fn = getattr(self.lib, f"{self.prefix}_set_num_threads", None)
        if fn is not None:
            fn.argtypes = [_I]
            fn(t)


_oracle = None
_ref = None


def oracle() -> CpuPath:
    """The restatement (always available once built)."""
    global _oracle
    if _oracle is None:
        if not os.path.exists(LIB_PATH):
            build(ref=False)
        _oracle = CpuPath(LIB_PATH, "oracle")
    return _oracle


def reference() -> CpuPath | None:
    """The compiled reference, or None when it was not built here."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        _ref = CpuPath(REF_PATH, "ref")
    return _ref


# --- the configs' input recipes (YTensor::seed + randn) ---

def bf16_inputs(path: CpuPath, seed: int, shapes, scales) -> list[np.ndarray]:
    """Draw each shape in order from one seeded stream, scale in fp32, round to
    bf16 with YTensor's rounding; returns uint16 bit arrays."""
    path.seed(seed)
    outs = []
    for shp, sc in zip(shapes, scales):
        x = path.randn(*shp)
        if sc != 1.0:
            x = (x * np.float32(sc)).astype(np.float32)
        outs.append(path.bf16_round(x))
    return outs


# --- Qwen3 configs[4] ------------------------------------------------------------

class Qwen3Config:
    """Qwen3Config defaults (example/qwen3/include/qwen3.hpp:46-60)."""

    def __init__(self, hidden=1024, layers=28, vocab=151936, inter=3072, n_heads=16, n_kv=8, head_dim=128,
                 max_pos=4096, eps=1e-6, theta=1e6):
        self.hidden, self.layers, self.vocab, self.inter = hidden, layers, vocab, inter
        self.n_heads, self.n_kv, self.head_dim, self.max_pos = n_heads, n_kv, head_dim, max_pos
        self.eps, self.theta = eps, theta


def qwen3_weight_layout(cfg: Qwen3Config) -> list[tuple[str, tuple[int, ...]]]:
    """(name, shape) in the fill order: embed, then per layer q, k, v, o,
    q_norm, k_norm, gate, up, down, norm1, norm2, then the final norm."""
    H, I, hd = cfg.hidden, cfg.inter, cfg.head_dim
    out = [("embed", (cfg.vocab, H))]
    for i in range(cfg.layers):
        out += [(f"{i}.q", (cfg.n_heads * hd, H)), (f"{i}.k", (cfg.n_kv * hd, H)), (f"{i}.v", (cfg.n_kv * hd, H)),
                (f"{i}.o", (H, cfg.n_heads * hd)), (f"{i}.q_norm", (hd,)), (f"{i}.k_norm", (hd,)),
                (f"{i}.gate", (I, H)), (f"{i}.up", (I, H)), (f"{i}.down", (H, I)),
                (f"{i}.norm1", (H,)), (f"{i}.norm2", (H,))]
    out.append(("norm", (H,)))
    return out


def qwen3_random_weights(path: CpuPath, cfg: Qwen3Config, seed: int = 3, scale: float = 0.02,
                         norm_spread: float | None = None) -> np.ndarray:
    """configs[4] init: YTensor::seed(seed), then every tensor randn * 0.02 in the
    layout order (norm weights included), rounded to bf16 and up-converted:
    returns the flat fp32 buffer of the bf16-representable weights.

    norm_spread: the discriminating variant -- the same stream, but every RMSNorm
    weight (q_norm, k_norm, norm1, norm2, final norm) is 1 + norm_spread * randn
    instead of randn * scale, so the activations keep their scale through the
    layers and the greedy stream moves from token to token."""
    path.seed(seed)
    total = sum(int(np.prod(s)) for _, s in qwen3_weight_layout(cfg))
    flat = np.empty(total, np.float32)
    off = 0
    for name, shp in qwen3_weight_layout(cfg):
        n = int(np.prod(shp))
        x = path.randn(n)
        if norm_spread is not None and "norm" in name:
            x = (np.float32(1.0) + x * np.float32(norm_spread)).astype(np.float32)
        else:
            x *= np.float32(scale)
        flat[off:off + n] = path.bf16_to_f32(path.bf16_round(x))
        off += n
    return flat


def qwen3_prompt(cfg: Qwen3Config, length: int = 512, seed: int = 4) -> np.ndarray:
    """Prompt tokens: std::mt19937(seed) + uniform_int_distribution[0, vocab-1]
    (the configs[4] recipe), drawn by numpy's MT19937 with the same seeding."""
    import random
    r = random.Random()
    # std::uniform_int_distribution's algorithm differs between libraries; the
    # recipe only needs a fixed, documented prompt, so a seeded Python stream is used.
    r.seed(seed)
    return np.array([r.randrange(cfg.vocab) for _ in range(length)], np.int32)
