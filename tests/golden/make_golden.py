"""Writes tests/golden/reference_host.npz: known answers of the reference's
own host-only code (oracle/_ref/libchimera_ref.so, built by oracle/Makefile
from the reference sources) on small seeded inputs.

Contents (all inputs are stored next to the outputs):
  flips_seed{S}                  FhtKac flip bytes for seed S (rotator.hpp:183-237)
  rot_in_d{D}, rot_out_d{D}      rotation of 16 vectors of dimension D with flips_seed42
  enc_in                         32 rotated unit vectors
  onebit_codes, onebit_factors   encode_one_bit (quantization.cpp:47-60)
  exq_b{B}                       quantize_ex codes, ex_bits B (quantization.cpp:121-146)
  full_b{B}, full_f_b{B}         encode_full_code packed codes and factors
  pack_raw_w{W}, pack_w{W}       packing_rabitqplus_code (pack_excode.hpp:274-297)
  unpack_w{W}                    select_excode_unpackfunc(W) output as float (W >= 2)
  gemv_q, gemv_x, gemv_out       gemv_batch8_avx512 with 32 queries
  fb_*                           compute_full_bit_scores loop (search_impl.cu:510-574)
                                 over a 16-document synthetic corpus, ex_bits 1..7

Usage: python tests/golden/make_golden.py   (needs oracle/_ref, i.e. the reference tree)
"""
from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as orc  # noqa: E402

P = C.c_void_p
OUT = Path(__file__).resolve().parent / "reference_host.npz"
TMP = b"/tmp/chimera_golden_flips.bin"


def ptr(a):
    return a.ctypes.data_as(P)


def main() -> None:
    ref = orc.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libchimera_ref.so is missing (run make -C oracle ref)")
    ref.ref_best_rescale_factor.restype = C.c_double
    rng = np.random.default_rng(20240601)
    g: dict[str, np.ndarray] = {}

    for seed in (42, 7, 123456789):
        f = np.zeros(64, np.uint8)
        assert ref.ref_rotator_flips(C.c_uint64(seed), 128, TMP, ptr(f)) == 0
        g[f"flips_seed{seed}"] = f
    flips = g["flips_seed42"]
    for d in (64, 96, 100, 128):
        x = rng.standard_normal((16, d)).astype(np.float32)
        y = np.zeros((16, 128), np.float32)
        assert ref.ref_rotate(d, ptr(flips), TMP, ptr(x), 16, ptr(y)) == 0
        g[f"rot_in_d{d}"] = x
        g[f"rot_out_d{d}"] = y

    x = rng.standard_normal((32, 128)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    enc = np.zeros((32, 128), np.float32)
    ref.ref_rotate(128, ptr(flips), TMP, ptr(x), 32, ptr(enc))
    g["enc_in"] = enc
    codes = np.zeros((32, 2), np.uint64)
    fac = np.zeros(32, np.float32)
    for i in range(32):
        f = C.c_float()
        ref.ref_encode_one_bit(ptr(enc[i]), ptr(codes[i]), C.byref(f))
        fac[i] = f.value
    g["onebit_codes"] = codes
    g["onebit_factors"] = fac
    for b in range(1, 8):
        exq = np.zeros((32, 128), np.uint8)
        full = np.zeros((32, 16 * (1 + b)), np.uint8)
        ff = np.zeros(32, np.float32)
        for i in range(32):
            ref.ref_quantize_ex(ptr(enc[i]), b, ptr(exq[i]))
            f = C.c_float()
            ref.ref_encode_full_code(ptr(enc[i]), b, ptr(full[i]), C.byref(f))
            ff[i] = f.value
        g[f"exq_b{b}"] = exq
        g[f"full_b{b}"] = full
        g[f"full_f_b{b}"] = ff

    for w in range(1, 9):
        raw = rng.integers(0, 1 << w, size=(8, 128)).astype(np.uint8)
        raw[0] = (1 << w) - 1
        raw[1] = 0
        pk = np.zeros((8, 16 * w), np.uint8)
        for i in range(8):
            ref.ref_pack(ptr(raw[i]), w, ptr(pk[i]))
        g[f"pack_raw_w{w}"] = raw
        g[f"pack_w{w}"] = pk
        if w >= 2:
            un = np.zeros((8, 128), np.float32)
            for i in range(8):
                ref.ref_unpack(ptr(pk[i]), w, ptr(un[i]))
            g[f"unpack_w{w}"] = un

    q = rng.standard_normal((32, 128)).astype(np.float32) * 0.1
    xv = rng.integers(0, 32, size=128).astype(np.float32)
    out = np.zeros(32, np.float32)
    ref.ref_gemv32(ptr(q), ptr(xv), ptr(out))
    g["gemv_q"], g["gemv_x"], g["gemv_out"] = q, xv, out

    # compute_full_bit_scores over a small corpus, every ex_bits
    lens = rng.integers(1, 20, size=16).astype(np.int32)
    ptrs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n = int(ptrs[-1])
    tok = rng.standard_normal((n, 128)).astype(np.float32)
    tok /= np.linalg.norm(tok, axis=1, keepdims=True)
    tok_rot = np.zeros_like(tok)
    ref.ref_rotate(128, ptr(flips), TMP, ptr(tok), n, ptr(tok_rot))
    qv = rng.standard_normal((32, 128)).astype(np.float32)
    qv /= np.linalg.norm(qv, axis=1, keepdims=True)
    q_rot = np.zeros_like(qv)
    ref.ref_rotate(128, ptr(flips), TMP, ptr(qv), 32, ptr(q_rot))
    g["fb_doc_ptrs"], g["fb_query_rot"] = ptrs, q_rot
    docs = np.arange(16, dtype=np.int32)
    for b in range(1, 8):
        codes = np.zeros((n, 16 * (1 + b)), np.uint8)
        facs = np.zeros(n, np.float32)
        for t in range(n):
            f = C.c_float()
            ref.ref_encode_full_code(ptr(tok_rot[t]), b, ptr(codes[t]), C.byref(f))
            facs[t] = f.value
        sumq = np.array([np.float32(0)] * 32, np.float32)
        cbex = np.zeros(32, np.float32)
        for i in range(32):
            s = np.float32(0)
            for j in range(128):
                s = np.float32(s + q_rot[i, j])
            sumq[i] = s
            cbex[i] = np.float32(np.float32(s * np.float32((1 << (b + 1)) - 1)) / np.float32(2.0))
        sc = np.zeros(16, np.float32)
        ref.ref_full_bit_scores(ptr(q_rot), ptr(cbex), ptr(ptrs), ptr(codes), ptr(facs), b, ptr(docs), 16, ptr(sc))
        g[f"fb_codes_b{b}"], g[f"fb_factors_b{b}"], g[f"fb_cbex_b{b}"], g[f"fb_scores_b{b}"] = codes, facs, cbex, sc

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(g)} arrays)")


if __name__ == "__main__":
    main()
