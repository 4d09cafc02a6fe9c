"""Writes tests/golden/ref_cpu_vectors.npz from the reference's own CPU path.

Run in the build container, where the reference sources exist:

    make -C oracle               # builds oracle/_ref/libkatali_ref.so from them
    python tests/golden/make_golden.py

Inputs are regenerated from seeds by tests/kq_synth.py; the fixture stores the
SHA-256 of every input so a changed generator fails loudly, and the reference
outputs as raw fp32 bit patterns:
  - katali_ggml_matvec (AVX2 row loop, hoisted Q4_K sums, dual rows)
    V/src/gguf_dtype.c:784-856 -> V/src/gguf_simd_x86.c:699-736,865-893
  - katali_ggml_vec_dot_ref (double accumulation), gguf_dtype.c:544-559
  - katali_ggml_vec_dot_scalar for Q4_K, gguf_dtype.c:594-624
  - katali_ggml_dequant_ref digest, gguf_dtype.c:429-512
  - katali_ggml_silu_mul_avx2, gguf_simd_x86.c:763-773
  - katali_gguf_softmax, gguf_kernels.c:74-80
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "tests"))

import kq_synth as S  # noqa: E402
from oracle import Q4_K, Q6_K, RefCPU  # noqa: E402

OUT = os.path.join(HERE, "ref_cpu_vectors.npz")

# (name, type, rows, cols, seed, fixed_scales)
MATVEC_CASES = [
    ("q4k_2048", Q4_K, 64, 2048, 101, False),
    ("q6k_768", Q6_K, 64, 768, 102, False),
    ("q4k_4096", Q4_K, 16, 4096, 103, False),
    ("q6k_12288", Q6_K, 8, 12288, 104, False),
    ("q6k_512", Q6_K, 32, 512, 105, False),
    ("q4k_1024_fixed", Q4_K, 25, 1024, 106, True),   # the reference tests' fill (d = dmin = 0.05)
    ("q6k_1024_fixed", Q6_K, 25, 1024, 107, True),
]


def case_inputs(t, rows, cols, seed, fixed):
    rng = np.random.default_rng(seed)
    w = S.fixed_scale_matrix(rng, t, rows, cols) if fixed else S.matrix(rng, t, rows, cols)
    x = S.activation(rng, cols)
    return w, x


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main() -> None:
    ref = RefCPU()
    assert ref.simd(), "the reference's AVX2 path must be active to record its fast-path outputs"
    out: dict[str, np.ndarray] = {}
    for name, t, rows, cols, seed, fixed in MATVEC_CASES:
        w, x = case_inputs(t, rows, cols, seed, fixed)
        out[f"{name}/input_sha256"] = np.array(sha(w, x))
        out[f"{name}/matvec"] = ref.matvec(t, w, rows, cols, x, threads=1, sums=True).view(np.uint32)
        out[f"{name}/vec_dot_ref"] = ref.vec_dot_rows(t, w, rows, cols, x, "ref").view(np.uint32)
        if t == Q4_K:
            out[f"{name}/vec_dot_scalar"] = ref.vec_dot_rows(t, w, rows, cols, x, "scalar").view(np.uint32)
        out[f"{name}/dequant_sha256"] = np.array(sha(ref.dequant(t, w, rows * cols)))
    rng = np.random.default_rng(201)
    g = (rng.standard_normal(768) * 4).astype(np.float32)
    u = rng.standard_normal(768).astype(np.float32)
    out["silu/input_sha256"] = np.array(sha(g, u))
    out["silu/out"] = ref.silu_mul(g, u).view(np.uint32)
    rng = np.random.default_rng(202)
    logits = rng.standard_normal(128).astype(np.float32)
    out["softmax/input_sha256"] = np.array(sha(logits))
    out["softmax/out"] = ref.softmax(logits).view(np.uint32)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
