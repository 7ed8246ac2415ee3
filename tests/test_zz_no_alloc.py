"""fo_contraction_noalloc (the entry point that allocates no device memory) against fo_contraction,
through the C ABI: bit-exact on two calls in a row, the second smaller (the static scratch keeps the
first call's contents), and a request beyond the 64 MiB static scratch is an error."""
import numpy as np
import pytest

import furiosa_hip as fh
from oracle import emulator as emu

pytestmark = pytest.mark.gpu

MAPS = ("M / 8, M % 8, K", "N, K", "M / 8, M % 8, N, K", "M / 8, M % 8, N")


def run_both(rt, M, N, K, in_t, out_t, seed):
    s = dict(M=M, N=N, K=K)
    rng = np.random.default_rng(seed)
    if in_t == fh.I4:
        a = rng.integers(0, 256, M * K // 2, dtype=np.uint8)
        b = rng.integers(0, 256, N * K // 2, dtype=np.uint8)
    else:
        a = emu.f32_to_bf16(rng.standard_normal(M * K).astype(np.float32))
        b = emu.f32_to_bf16(rng.standard_normal(N * K).astype(np.float32))
    ob = {fh.I4: 1, fh.I32: 4, fh.BF16: 2}[out_t]
    nbytes = M * N * ob // (2 if out_t == fh.I4 else 1)
    da, db = rt.upload(a), rt.upload(b)
    maps = [fh.m(t, **s) for t in MAPS]
    ref, got = rt.alloc(nbytes), rt.alloc(nbytes)
    rt.contraction(ref, da, db, in_t, out_t, *maps)
    rt.contraction_noalloc(got, da, db, in_t, out_t, *maps)
    np_t = np.uint8 if out_t == fh.I4 else fh.NP_DTYPE[out_t]
    return got.read(np_t), ref.read(np_t)


@pytest.mark.parametrize("out_t", [fh.I32, fh.I4], ids=["i4_to_i32", "i4_to_i4"])
def test_noalloc_matches_contraction_twice(rt, out_t):
    # first call large (8 MiB / 24 MiB of scratch), the second smaller (reuses the array)
    for (M, N, K), seed in (((2048, 2048, 2048), 1), ((256, 384, 512), 2)):
        got, ref = run_both(rt, M, N, K, fh.I4, out_t, seed)
        assert np.array_equal(got, ref), (M, N, K)


def test_noalloc_non_i4_types_match(rt):
    got, ref = run_both(rt, 512, 256, 384, fh.BF16, fh.BF16, 3)
    assert np.array_equal(got, ref)


def test_noalloc_rejects_beyond_the_static_scratch(rt):
    # i4 -> i4 at 4096^3: 16 MiB + 16 MiB unpacked operands + 64 MiB i32 staging > 64 MiB
    s = dict(M=4096, N=4096, K=4096)
    a = rt.alloc(4096 * 4096 // 2)
    out = rt.alloc(4096 * 4096 // 2)
    with pytest.raises(fh.FoError, match="64 MiB static scratch"):
        rt.contraction_noalloc(out, a, a, fh.I4, fh.I4, *(fh.m(t, **s) for t in MAPS))
