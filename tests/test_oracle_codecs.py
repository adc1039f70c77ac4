"""Pins the oracle's number codecs against independent implementations.

binary16: numpy's float16 (exhaustive decode, random encode).
E4M3: torch.float8_e4m3fn's decode table and encoder (golden fixtures written
by tests/golden/make_golden.py), plus properties the OCP definition fixes.
"""

import pathlib

import numpy as np

import oracle

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def test_f16_decode_all_codes_match_numpy():
    h = np.arange(65536, dtype=np.uint16)
    ours = oracle.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    assert np.array_equal(ours[~np.isnan(ref)], ref[~np.isnan(ref)])


def test_f16_encode_matches_numpy_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32),
        (rng.standard_normal(200000) * 3e4).astype(np.float32),
        (rng.standard_normal(200000) * 1e-6).astype(np.float32),          # subnormals
        np.array([65504, 65519.99, 65520, 7e4, np.inf, -np.inf, 0.0, -0.0], np.float32),
    ])
    # exact halfway points between neighbouring fp16 values (ties to even)
    h = np.arange(0, 0x7bff, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    x = np.concatenate([x, ((lo + hi) / 2).astype(np.float32)])
    with np.errstate(over="ignore"):   # values past 65519.99 round to inf on purpose
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16_bits(x), want)


def test_e4m3_decode_matches_torch_table():
    ref = np.load(GOLDEN / "e4m3_decode.npy")
    ours = oracle.e4m3_to_f32(np.arange(256))
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    assert np.array_equal(ours[~np.isnan(ref)], ref[~np.isnan(ref)])
    # OCP E4M3: max normal 448, NaN only at S.1111.111, min subnormal 2^-9
    assert ours[0x7E] == 448.0 and np.isnan(ours[0x7F]) and np.isnan(ours[0xFF])
    assert ours[1] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6


def test_e4m3_encode_matches_torch_vectors():
    g = np.load(GOLDEN / "e4m3_encode.npz")
    assert np.array_equal(oracle.f32_to_e4m3(g["x"]), g["code"])


def test_e4m3_encode_properties():
    vals = oracle.e4m3_to_f32(np.arange(0x7F))
    # every finite code round-trips, both signs
    assert np.array_equal(oracle.f32_to_e4m3(vals), np.arange(0x7F, dtype=np.uint8))
    assert np.array_equal(oracle.f32_to_e4m3(-vals[1:]), (np.arange(1, 0x7F) | 0x80).astype(np.uint8))
    # midpoints go to the even code; just off a midpoint goes to the nearer code
    mids = ((vals[1:].astype(np.float64) + vals[:-1]) / 2).astype(np.float32)
    codes = oracle.f32_to_e4m3(mids)
    lower = np.arange(0x7E)
    assert np.array_equal(codes, np.where(lower % 2 == 0, lower, lower + 1).astype(np.uint8))
    up = np.nextafter(mids, np.float32(np.inf))
    assert np.array_equal(oracle.f32_to_e4m3(up), (lower + 1).astype(np.uint8))
    # saturation (satfinite) for overflow and infinity, NaN preserved
    big = np.array([448, 449, 463.9, 464, 480, 1e6, np.inf], np.float32)
    assert np.all(oracle.f32_to_e4m3(big) == 0x7E)
    assert np.all(oracle.f32_to_e4m3(-big) == 0xFE)
    assert oracle.f32_to_e4m3(np.array([np.nan], np.float32))[0] & 0x7F == 0x7F
    # monotone over a dense sweep
    x = np.linspace(-500, 500, 100001, dtype=np.float32)
    v = oracle.e4m3_to_f32(oracle.f32_to_e4m3(x))
    assert np.all(np.diff(v) >= 0)
