"""Write the .yt fixtures under tests/golden/ with the COMPILED REFERENCE's
yt::io::YTensorIO (oracle/_ref/libytref.so, built from /root/reference by
`make -C oracle ref`; runs only where the reference exists).

    python tests/golden/make_yt_fixtures.py

Files (every byte written by the reference):
  yt_plain.yt    the tensors of `tensors()` below, no compression (Write)
  yt_zlib.yt     the same, yt::io::compressMethod = "zlib"
  yt_base.yt     a (float32 [4]), b (bfloat16 [8]), c (int32 [3])
  yt_append.yt   yt_base.yt, then open(Append): save(c2 as "c"), save(d), save(e, "")
  yt_rewrite.yt  yt_base.yt, then open(Write):  save(c2 as "c"), save(e, ""), save(a2 as "a")
  yt_expected.npz  per tensor of yt_plain.yt: what YTensorIO::load returned
                   (typeName, shape, raw bytes), read back through the reference
The inputs are small deterministic arrays (numpy seeds below) plus hand-picked
special values (NaN payloads, infinities, signed zeros, subnormals, fp16
overflow and underflow, bf16 / fp16 rounding ties).
"""
from __future__ import annotations

import os
import shutil
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

SPECIAL_F32_BITS = [
    0x00000000, 0x80000000, 0x3F800000, 0xBF800000, 0x7FC00000, 0x7F800001, 0xFFC12345, 0x7F800000,
    0xFF800000, 0x00000001, 0x006CE3EE,   # fp32 subnormals
    0x477FE000, 0x477FF000, 0x47800000,   # 65504, 65520 (fp16 rounds to inf), 65536
    0x33000000, 0x38800000, 0x387FC000,   # 2^-25 (fp16 underflow), 2^-14 (fp16 min normal), just below
    0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F807FFF,  # bf16: ties with bit16 = 0 / 1, near ties
    0x3F801000, 0x3F803000, 0x3F801001,   # fp16: ties to even (down / up), just above a tie
]
SPECIAL_F16_BITS = [0x0000, 0x8000, 0x0001, 0x03FF, 0x8200, 0x0400, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00,
                    0x7C01, 0x3C00, 0x3555, 0x1234]


def tensors() -> list[tuple[str, str, list[int], np.ndarray]]:
    # inputs are rounded with the oracle's casts (pinned bit-exact to the
    # reference's by tests/test_oracle.py) so that tests can rebuild them anywhere
    ref = oracle.oracle()
    rng = np.random.default_rng(20)
    w = ref.bf16_round((rng.standard_normal((24, 40)) * 0.02).astype(np.float32))
    f16 = ref.f16_round(rng.standard_normal(3 * 5 * 7 - len(SPECIAL_F16_BITS)).astype(np.float32))
    f16 = np.concatenate([np.array(SPECIAL_F16_BITS, np.uint16), f16]).reshape(3, 5, 7)
    return [
        ("model.layers.0.self_attn.q_proj.weight", "bfloat16", [24, 40], w),
        ("model.norm.weight", "float32", [40], (1 + 0.1 * rng.standard_normal(40)).astype(np.float32)),
        ("act_f16", "float16", [3, 5, 7], f16),
        ("ids", "int32", [10], rng.integers(-2**31, 2**31 - 1, 10, dtype=np.int64).astype(np.int32)),
        ("scale", "float64", [], np.array([0.08838834764831845], np.float64)),
        ("special_f32", "float32", [len(SPECIAL_F32_BITS)], np.array(SPECIAL_F32_BITS, np.uint32).view(np.float32)),
        ("big_f32", "float32", [300, 7], rng.standard_normal((300, 7)).astype(np.float32)),
        ("bytes_u8", "uint8", [2, 3, 4], np.arange(24, dtype=np.uint8)),
    ]


def base_set():
    rng = np.random.default_rng(21)
    a = rng.standard_normal(4).astype(np.float32)
    b = oracle.oracle().bf16_round(rng.standard_normal(8).astype(np.float32))
    c = np.array([7, -8, 9], np.int32)
    return [("a", "float32", [4], a), ("b", "bfloat16", [8], b), ("c", "int32", [3], c)]


def update_sets():
    """The tensors saved over yt_base.yt: (append list, rewrite list)."""
    rng = np.random.default_rng(22)
    c2 = rng.standard_normal(2).astype(np.float32)
    d = oracle.oracle().f16_round(rng.standard_normal(5).astype(np.float32))
    e = np.array([3.5], np.float32)
    a2 = rng.standard_normal((2, 3)).astype(np.float32)
    append = [("c", "float32", [2], c2), ("d", "float16", [5], d), ("", "float32", [1], e)]
    rewrite = [("c", "float32", [2], c2), ("", "float32", [1], e), ("a", "float32", [2, 3], a2)]
    return append, rewrite


def main() -> None:
    ref = oracle.reference()
    if ref is None:
        raise SystemExit("oracle/_ref/libytref.so is not built (make -C oracle ref)")
    ts = tensors()
    p = lambda n: os.path.join(HERE, n)  # noqa: E731
    ref.yt_save(p("yt_plain.yt"), ts)
    ref.yt_save(p("yt_zlib.yt"), ts, "zlib")
    ref.yt_save(p("yt_base.yt"), base_set())
    app, rew = update_sets()
    shutil.copy(p("yt_base.yt"), p("yt_append.yt"))
    ref.yt_save(p("yt_append.yt"), app, "", mode=3)
    shutil.copy(p("yt_base.yt"), p("yt_rewrite.yt"))
    ref.yt_save(p("yt_rewrite.yt"), rew, "", mode=2)
    exp = {}
    for name, _, _, _ in ts:
        tname, shape, raw = ref.yt_load(p("yt_plain.yt"), name)
        exp[f"{name}|type"] = np.array(tname)
        exp[f"{name}|shape"] = np.array(shape, np.int64)
        exp[f"{name}|bytes"] = np.frombuffer(raw, np.uint8)
    exp["names_append"] = np.array(ref.yt_names(p("yt_append.yt")))
    exp["names_rewrite"] = np.array(ref.yt_names(p("yt_rewrite.yt")))
    np.savez(p("yt_expected.npz"), **exp)
    for n in ("yt_plain.yt", "yt_zlib.yt", "yt_base.yt", "yt_append.yt", "yt_rewrite.yt", "yt_expected.npz"):
        print(n, os.path.getsize(p(n)))


if __name__ == "__main__":
    main()
