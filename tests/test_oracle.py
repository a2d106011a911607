"""Pins of the CPU oracle (oracle/exl3_oracle.c) — CPU only.

Each oracle function is checked against something it does not restate:
  * golden vectors written from the reference's own compiled decode header
    (tests/golden/make_golden.py): codebook tables, windows, composed dequant;
  * the reference header itself when oracle/_ref is built (exhaustive);
  * closed forms: all-zero trellis, single-window tiles, Sylvester-matrix FWHT,
    W = suh (.) svh (.) (H T H)/128 by numpy matrix products;
  * brute force on tiny inputs (bit-serial window reader).
"""

import hashlib
import os

import numpy as np
import pytest

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _f16(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


# ------------------------------------------------------------------ codebooks

@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_table_matches_reference_digest(cb):
    g = np.load(os.path.join(GOLD, "codebooks.npz"))
    table = oracle.codebook_table(cb, rtz=True)
    assert hashlib.sha256(table.tobytes()).digest() == g[f"sha256_cb{cb}"].tobytes()
    assert np.array_equal(table[g[f"states_cb{cb}"]], g[f"bits_cb{cb}"])


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_exhaustive_vs_reference_header(cb):
    R = oracle.ref_lib()
    if R is None:
        pytest.skip("reference header not built here")
    ref = np.array([R.ref_decode_codebook_bits(s, cb) for s in range(65536)], dtype=np.uint16)
    assert np.array_equal(oracle.codebook_table(cb, rtz=True), ref)


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_rne_and_rtz_tables_bracket_the_exact_value(cb):
    """Both tables round the same exact value: RTZ truncates toward 0,
    RNE is the nearest fp16; they agree wherever the exact value is an fp16."""
    exact = np.array([oracle.lib().orc_codebook_exact(s, cb) for s in range(0, 65536, 7)], dtype=np.float64)
    rtz = _f16(oracle.codebook_table(cb, rtz=True)[::7])
    rne = _f16(oracle.codebook_table(cb, rtz=False)[::7])
    assert np.all(np.abs(rtz) <= np.abs(exact))
    assert np.all(np.abs(rne - exact) <= np.abs(rtz - exact))
    rep = exact.astype(np.float16).astype(np.float64) == exact
    assert np.array_equal(rtz[rep], rne[rep])
    ulp = np.spacing(np.abs(rtz).astype(np.float16)).astype(np.float64)  # upward from |rtz|
    assert np.all(np.abs(rtz - exact) < ulp)


def test_codebook_state_zero_closed_form():
    """state 0: MCG -> 0x3b60 + 0x3b60 = 1.84375; mul1 -> 1024 * 0x1eee + 0xc931 = -3.453125."""
    assert _f16(oracle.codebook_table(1, True)[0]) == 1.84375
    assert _f16(oracle.codebook_table(2, True)[0]) == -3.453125


def test_mul1_codebook_formula_by_integers():
    """mul1 value = ((0x6400 + byte_sum(s*M)) as fp16) * 0x1eee + 0xc931, evaluated in exact
    integer arithmetic: (1024 + S) * 1774 * 2^-18 - 2721792 * 2^-18."""
    for s in range(0, 65536, 97):
        x = (s * 0x83DCD12D) & 0xFFFFFFFF
        S = sum((x >> (8 * i)) & 255 for i in range(4))
        exact = ((1024 + S) * 1774 - 2721792) / 262144.0
        assert oracle.lib().orc_codebook_exact(s, 2) == pytest.approx(exact, abs=0, rel=0)


# -------------------------------------------------------------------- windows

@pytest.mark.parametrize("K", range(1, 9))
def test_read_window_matches_golden(K):
    g = np.load(os.path.join(GOLD, "windows.npz"))
    tile = g[f"tile_K{K}"]
    got = np.array([oracle.read_window(tile, b) for b in range(256 * K)], dtype=np.uint16)
    assert np.array_equal(got, g[f"win_K{K}"])


@pytest.mark.parametrize("K", [1, 3, 4, 7])
def test_read_window_brute_force_bitstream(K):
    """16 bits starting at stream bit b of the cyclic MSB-first stream of LE uint32 words."""
    rng = np.random.default_rng(K)
    tile = rng.integers(0, 65536, size=16 * K, dtype=np.uint16)
    words = tile.view(np.uint32)
    bits = np.array([(int(w) >> (31 - i)) & 1 for w in words for i in range(32)], dtype=np.int64)
    for b in range(0, 256 * K, 5):
        want = 0
        for i in range(16):
            want = (want << 1) | int(bits[(b + i) % bits.size])
        assert oracle.read_window(tile, b) == want


# ----------------------------------------------------------------- tile layout

@pytest.mark.parametrize("cb", [1, 2])
def test_tile_layout_single_window(cb):
    """A tile with exactly one value's window set to a distinct state: the decoded tile
    differs from the all-zero tile at the one position the closed-form layout gives."""
    K = 4
    base = oracle.decode_tile(np.zeros(16 * K, dtype=np.uint16), K, cb, rtz=True)
    for t in (0, 1, 7, 8, 37, 128, 200, 255):
        # value t's window ends at bit (t+1)K: set the low bit of that window only
        tile = np.zeros(16 * K, dtype=np.uint16)
        bit = ((t + 1) * K - 1) % (256 * K)
        word, off = divmod(bit, 32)
        w = tile.view(np.uint32)
        w[word] |= np.uint32(1 << (31 - off))
        dec = oracle.decode_tile(tile, K, cb, rtz=True)
        diff = np.argwhere(dec != base)
        l, j = divmod(t, 8)
        want_k = 2 * (l % 4) + (j & 1) + 8 * ((j >> 1) & 1)
        want_n = l // 4 + 8 * (j >> 2)
        # the window of value t contains that bit as its LSB; the next values' windows
        # contain it too (shifted), so the changed set starts at t
        assert [want_k, want_n] in diff.tolist()


# --------------------------------------------------------------- hadamard

def _sylvester(n):
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


def test_fwht_is_sylvester_product_and_involution():
    rng = np.random.default_rng(3)
    v = rng.standard_normal(128).astype(np.float32)
    H = _sylvester(128)
    assert np.allclose(oracle.fwht(v), H @ v.astype(np.float64), rtol=1e-5, atol=1e-4)
    back = oracle.fwht(oracle.fwht(v)) / 128.0
    assert np.allclose(back, v, atol=1e-5)


def test_fwht_matches_reference_header_bitwise():
    R = oracle.ref_lib()
    if R is None:
        pytest.skip("reference header not built here")
    rng = np.random.default_rng(4)
    for _ in range(20):
        v = rng.standard_normal(128).astype(np.float32)
        b = v.copy()
        R.ref_hadamard(b.ctypes.data, 128)
        assert np.array_equal(oracle.fwht(v).view(np.uint32), b.view(np.uint32))


# ------------------------------------------- transform_hadamard_fast (had_fast)

def test_round_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(11)
    a = (rng.standard_normal(4096) * np.exp2(rng.integers(-20, 20, 4096))).astype(np.float32)
    # exact ties: bit 15 set, bits 0..14 clear, both parities of bit 16
    ties = (a.view(np.uint32) & np.uint32(0xFFFF0000)) | np.uint32(0x8000)
    a = np.concatenate([a, ties.view(np.float32), np.float32([0.0, -0.0, 1.0, -3.5])])
    want = torch.from_numpy(a).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(oracle.round_bf16(a).view(np.uint32), want.view(np.uint32))


def test_sylvester_matches_fwht():
    H = oracle.sylvester(128)
    assert np.array_equal(H, _sylvester(128))
    e = np.eye(128, dtype=np.float32)
    assert np.array_equal(np.stack([oracle.fwht(r) for r in e]), H.astype(np.float32))


@pytest.mark.parametrize("dtype,h", [("f16", 181 / 2048), ("bf16", 181 / 2048), ("f32", float(np.float32(0.08838834764831845)))])
def test_had_fast_one_hot_and_constant_rows(dtype, h):
    """One-hot row i gives +-h in column j with the sign of H[i][j] (exactly the
    dtype's 1/sqrt(128)); a row of ones gives T(128 h) in column 0 of each block
    and zeros elsewhere."""
    H = oracle.sylvester(128)
    x = np.eye(256, dtype=np.float32)[:256:37]
    y = oracle.had_fast(x, None, dtype)
    for r, i in enumerate(range(0, 256, 37)):
        blk = i // 128
        want = np.zeros(256)
        want[blk * 128:(blk + 1) * 128] = H[i % 128] * h
        assert np.array_equal(y[r], want.astype(np.float32))
    ones = oracle.had_fast(np.ones((1, 256), np.float32), None, dtype)
    want = np.zeros(256, np.float32)
    want[[0, 128]] = oracle.round_to(np.float32(128 * h), dtype)
    assert np.array_equal(ones[0], want)


def test_had_fast_rounds_twice_around_post():
    """x = 3 e_0, post[0] = p: y[0] = T(T(3h) p), not T(3h p) (two roundings,
    the reference's matmul output and then its suh product)."""
    h = 181 / 2048
    p = np.float16(1.0009765625)  # 1 + 2^-10
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = 3.0
    post = np.ones(128, np.float16)
    post[0] = p
    y = oracle.had_fast(x, post, "f16")
    t = np.float16(np.float32(3 * h))
    assert y[0, 0] == np.float16(np.float32(t) * np.float32(p))
    assert np.array_equal(y[0, 1:], np.float32(t) * oracle.sylvester(128)[0, 1:].astype(np.float32))


def test_had_fast_is_near_involution_in_f32():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((3, 384)).astype(np.float32)
    back = oracle.had_fast(oracle.had_fast(x, None, "f32"), None, "f32")
    assert np.allclose(back, x, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------- dequant

@pytest.mark.parametrize("tag", ["K2_mcg", "K3_mul1", "K4_mcg", "K4_mul1", "K5_mcg", "K8_mul1"])
def test_dequant_matches_golden_bits(tag):
    g = np.load(os.path.join(GOLD, "dequant.npz"))
    K = int(tag[1])
    cb = 1 if tag.endswith("mcg") else 2
    W = oracle.dequant(g[f"trellis_{tag}"], g[f"suh_{tag}"], g[f"svh_{tag}"], K, cb, rtz=True)
    assert np.array_equal(W, g[f"W_{tag}"])


def test_dequant_equals_matrix_form():
    """W = suh (.) svh (.) (H T H) / 128 per 128-block, computed by dense matrix products
    in float64 (a different algorithm); agreement within fp16 rounding."""
    K, cb = 3, 1
    rng = np.random.default_rng(9)
    k, n = 256, 128
    tr = rng.integers(0, 65536, size=(k // 16, n // 16, 16 * K), dtype=np.uint16)
    su = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
    sv = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
    T = np.zeros((k, n))
    for kt in range(k // 16):
        for nt in range(n // 16):
            T[kt * 16:(kt + 1) * 16, nt * 16:(nt + 1) * 16] = _f16(oracle.decode_tile(tr[kt, nt], K, cb, rtz=True))
    H = _sylvester(128)
    Wm = np.zeros((k, n))
    for r0 in range(0, k, 128):
        for c0 in range(0, n, 128):
            Wm[r0:r0 + 128, c0:c0 + 128] = H @ T[r0:r0 + 128, c0:c0 + 128] @ H / 128.0
    Wm *= su.astype(np.float64)[:, None] * sv.astype(np.float64)[None, :]
    W = _f16(oracle.dequant(tr, su, sv, K, cb, rtz=True))
    assert np.max(np.abs(W - Wm)) <= 2.0 ** -10 * np.max(np.abs(Wm)) + 1e-6


def test_dequant_all_zero_trellis_closed_form():
    """Reference fixture (tests/test_cuda_graph.py:76-78) at a dequant-valid size:
    W = 128 c suh svh at each (128i, 128j) corner, 0 elsewhere."""
    for cb, c in ((1, 1.84375), (2, -3.453125)):
        k, n = 256, 384
        rng = np.random.default_rng(2)
        su = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
        sv = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
        W = _f16(oracle.dequant(np.zeros((k // 16, n // 16, 32), dtype=np.uint16), su, sv, 2, cb, rtz=True))
        corner = W[::128, ::128]
        want = 128.0 * c * np.outer(su[::128].astype(np.float64), sv[::128].astype(np.float64))
        assert np.allclose(corner, want, rtol=1e-3)
        mask = np.ones_like(W, dtype=bool)
        mask[::128, ::128] = False
        assert np.all(W[mask] == 0.0)


def test_cpu_gemv_is_dequant_then_fp32_product():
    rng = np.random.default_rng(1)
    k, n, K = 256, 256, 4
    tr = rng.integers(0, 65536, size=(k // 16, n // 16, 16 * K), dtype=np.uint16)
    su = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
    sv = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
    x = rng.standard_normal((2, k)).astype(np.float16)
    y = oracle.cpu_gemv(x, tr, su, sv, K, 1)
    W = _f16(oracle.dequant(tr, su, sv, K, 1, rtz=True))
    assert np.allclose(y, x.astype(np.float64) @ W, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("m,k,n", [(1, 256, 384), (3, 640, 128), (17, 96, 200)])
def test_matmul_matches_float64_numpy_product(m, k, n):
    """oracle.matmul against numpy's float64 product of the same fp16 operands
    (a different summation order and code).  Each fp16 x fp16 product is exact,
    so the only error is fp64 accumulation (<= k eps64 sum|x||W|) plus the final
    fp32 rounding (half an fp32 ulp).  k != n, so a transposed operand fails."""
    rng = np.random.default_rng(100 + m)
    x = rng.standard_normal((m, k)).astype(np.float16)
    W = (rng.standard_normal((k, n)) * 3).astype(np.float16)
    want = x.astype(np.float64) @ W.astype(np.float64)
    got = oracle.matmul(x, W).astype(np.float64)
    mag = np.abs(x.astype(np.float64)) @ np.abs(W.astype(np.float64))
    bound = 0.5 * np.spacing(np.abs(want).astype(np.float32)).astype(np.float64) + k * 2.0 ** -52 * mag
    assert np.all(np.abs(got - want) <= bound)


def test_matmul_one_hot_rows_select_weight_rows():
    """x = e_i gives y = W[i, :] exactly; x = a e_i + b e_j gives a W_i + b W_j
    (exact here: power-of-two coefficients)."""
    rng = np.random.default_rng(21)
    k, n = 48, 80
    W = rng.standard_normal((k, n)).astype(np.float16)
    idx = [0, 7, 47, 13]
    x = np.zeros((len(idx) + 1, k), dtype=np.float16)
    for r, i in enumerate(idx):
        x[r, i] = 1.0
    x[-1, 3], x[-1, 30] = 2.0, -0.25
    y = oracle.matmul(x, W)
    for r, i in enumerate(idx):
        assert np.array_equal(y[r], W[i].astype(np.float32))
    Wd = W.astype(np.float64)
    assert np.array_equal(y[-1].astype(np.float64), 2.0 * Wd[3] - 0.25 * Wd[30])


def test_matmul_propagates_inf_and_nan_like_ieee():
    """A zero input times an inf or NaN weight is NaN (no zero-input shortcut);
    a finite input times inf is inf; numpy's float64 product is the check."""
    k, n = 8, 6
    W = np.ones((k, n), dtype=np.float16)
    W[2, 1] = np.inf
    W[5, 4] = np.nan
    x = np.ones((3, k), dtype=np.float16)
    x[1, 2] = 0.0
    x[2, 5] = 0.0
    x[2, 2] = -1.0
    with np.errstate(invalid="ignore"):
        want = x.astype(np.float64) @ W.astype(np.float64)
    got = oracle.matmul(x, W).astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin], want[fin])
    assert np.isnan(got[1, 1]) and np.isnan(got[2, 4]) and got[2, 1] == -np.inf


@pytest.mark.parametrize("cb,c", [(1, 1.84375), (2, -3.453125)])
def test_linear_ref_zero_trellis_closed_form(cb, c):
    """All-zero trellis through linear_ref (dequant then matmul): only the
    (128i, 128j) corners of W are non-zero, so
    y[128j] = 128 c svh[128j] sum_i x[128i] suh[128i] and y = 0 elsewhere."""
    k, n, K = 384, 256, 3
    rng = np.random.default_rng(31 + cb)
    su = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
    sv = (np.where(rng.random(n) < 0.5, -1.0, 1.0) * 2.0 ** rng.integers(-2, 3, n)).astype(np.float16)
    x = rng.standard_normal((5, k)).astype(np.float16)
    y = oracle.linear_ref(x, np.zeros((k // 16, n // 16, 16 * K), dtype=np.int16), su, sv, K, cb).astype(np.float64)
    s = (x[:, ::128].astype(np.float64) * su[::128].astype(np.float64)).sum(axis=1)
    want = 128.0 * c * np.outer(s, sv[::128].astype(np.float64))
    assert np.allclose(y[:, ::128], want, rtol=1e-6, atol=0)
    mask = np.ones(n, dtype=bool)
    mask[::128] = False
    assert not y[:, mask].any()


def test_swiglu_matches_torch_silu():
    """oracle.swiglu against torch's own SiLU (an independent implementation of
    silu(min(g, L)) * clamp(u, -L, L), src/sglang_exl3/exl3.py:572), on values
    from the saturated tails through zero; and the C restatement agrees too."""
    import torch

    rng = np.random.default_rng(12)
    g = np.concatenate([rng.standard_normal(4000) * 6, [-80.0, -20.0, -1e-3, 0.0, 1e-3, 20.0, 80.0]]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32) * 3
    for L in (float("inf"), 0.0, 1.0, 4.5):
        gt, ut = torch.from_numpy(g.astype(np.float64)), torch.from_numpy(u.astype(np.float64))
        if L > 0 and np.isfinite(L):
            gt, ut = gt.clamp(max=L), ut.clamp(min=-L, max=L)
        want = (torch.nn.functional.silu(gt) * ut).numpy()
        got = oracle.swiglu(g, u, L)
        assert np.allclose(got, want, rtol=2e-6, atol=1e-30), f"limit {L}"
    for gi, ui in zip(g[::400], u[::400]):
        want = float(torch.nn.functional.silu(torch.tensor(float(gi), dtype=torch.float64)) * float(ui))
        assert oracle.lib().orc_swiglu(float(gi), float(ui), 0.0) == pytest.approx(want, rel=2e-6, abs=1e-30)


def _tiny_experts(E, hidden, inter, K, seed):
    out = []
    for e in range(E):
        spec = {}
        for j, (proj, k, n) in enumerate((("gate", hidden, inter), ("up", hidden, inter), ("down", inter, hidden))):
            r = np.random.default_rng(seed + 3 * e + j)
            tr = r.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int64).astype(np.int16)
            su = np.where(r.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
            sv = (np.where(r.random(n) < 0.5, -1.0, 1.0) * (4.0 / np.sqrt(k))).astype(np.float16)
            spec[proj] = (tr, su, sv, K, 1)
        out.append(spec)
    return out


def test_moe_ref_reduces_to_composed_linears():
    """Top-1 routing with weight 1 is down(swiglu(gate x, up x)) of that expert,
    built from linear_ref; invalid ids contribute nothing."""
    E, H, I, K = 3, 128, 128, 2
    experts = _tiny_experts(E, H, I, K, seed=5)
    x = np.random.default_rng(6).standard_normal((4, H)).astype(np.float16)
    ids = np.array([[2], [0], [1], [-1]], dtype=np.int32)
    w = np.ones((4, 1), dtype=np.float32)
    got = oracle.moe_ref(x, ids, w, experts)
    for t in range(3):
        ex = experts[int(ids[t, 0])]
        g = oracle.linear_ref(x[t:t + 1], *ex["gate"])
        u = oracle.linear_ref(x[t:t + 1], *ex["up"])
        act = oracle.swiglu(g, u, float("inf")).astype(np.float16)
        want = oracle.linear_ref(act, *ex["down"])
        assert np.array_equal(got[t], want[0])
    assert not got[3].any()


def test_moe_ref_is_linear_in_the_routing_weights():
    """Doubling every routing weight doubles the output; two slots add up to the
    sum of the one-slot outputs."""
    E, H, I, K = 4, 128, 128, 3
    experts = _tiny_experts(E, H, I, K, seed=9)
    rng = np.random.default_rng(10)
    x = rng.standard_normal((5, H)).astype(np.float16)
    ids = np.stack([rng.choice(E, 2, replace=False) for _ in range(5)]).astype(np.int32)
    w = rng.random((5, 2)).astype(np.float32)
    base = oracle.moe_ref(x, ids, w, experts)
    assert np.allclose(oracle.moe_ref(x, ids, 2 * w, experts), 2 * base, rtol=1e-6, atol=1e-6)
    one = oracle.moe_ref(x, ids[:, :1], w[:, :1], experts) + oracle.moe_ref(x, ids[:, 1:], w[:, 1:], experts)
    assert np.allclose(base, one, rtol=1e-5, atol=1e-5)