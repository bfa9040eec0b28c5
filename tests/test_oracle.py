"""Pins the CPU oracle (oracle/kf_oracle.c) before anything is checked against it.

Each check is chosen so that a plausible mistake in the restatement (a dropped term, a wrong nibble or scale index, a
swapped rounding mode, a wrong sign of the min term) fails it:
  * the reference's own golden vectors: ggml-produced dequant outputs, bit-exact
    (crates/kf-quant/tests/fixtures/{q8_0,q4_K,q8_K}.bin, checked as crates/kf-quant/tests/parity.rs:106-130);
  * the reference's own invariants, restated with its RNG and seeds (parity.rs:132-167 dot_row, :169-203 dot_i8);
  * numpy's IEEE binary16 conversion for the f16 boundary (the `half` crate is not importable here);
  * closed forms and brute force: integer block dots from numpy int64 arithmetic, the q4_K special case that reduces
    to a textbook integer dot, hand-made rounding ties, and the float product against float64 numpy.
"""
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


class SplitMix:
    """The RNG of crates/kf-quant/tests/parity.rs:75-88."""

    def __init__(self, seed):
        self.s = seed & 0xFFFFFFFFFFFFFFFF

    def next(self):
        M = 0xFFFFFFFFFFFFFFFF
        self.s = (self.s + 0x9E3779B97F4A7C15) & M
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return z ^ (z >> 31)

    def unit(self):
        return np.float32((self.next() >> 40) / float(1 << 24))


# ------------------------------------------------------------------ layouts and golden vectors

def test_layouts_match_ggml_structs():
    # parity.rs:9-31 (q4_K, q8_K) and q8_0.rs:4
    import ctypes

    for ty, want in [(8, (32, 34)), (12, (256, 144)), (13, (256, 176)), (14, (256, 210)), (15, (256, 292))]:
        b, s = ctypes.c_int(), ctypes.c_int()
        assert oracle.lib().kfo_type_info(ty, ctypes.byref(b), ctypes.byref(s)) == 0
        assert (b.value, s.value) == want
    assert oracle.lib().kfo_type_info(2, ctypes.byref(b), ctypes.byref(s)) == -1


ALL_FIXTURES = [("q8_0", 8), ("q4_K", 12), ("q5_K", 13), ("q6_K", 14), ("q8_K", 15)]


@pytest.mark.parametrize("name,ty", ALL_FIXTURES)
def test_fixture_rows_match_type_size(name, ty):
    n, rows, blocks, _ = oracle.load_fixture(os.path.join(GOLDEN, f"{name}.bin"))
    assert blocks.size == rows * oracle.row_bytes(ty, n)


@pytest.mark.parametrize("name,ty", ALL_FIXTURES)
def test_dequant_is_bit_exact_with_ggml(name, ty):
    n, rows, blocks, want = oracle.load_fixture(os.path.join(GOLDEN, f"{name}.bin"))
    got = oracle.dequant(ty, blocks, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------ f16 (half 2.7.1) against numpy's binary16

def test_f16_to_f32_exhaustive():
    L = oracle.lib()
    h = np.arange(65536, dtype=np.uint32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([L.kfo_f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_trip_and_ties():
    L = oracle.lib()
    finite = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    fv = finite.view(np.float16)
    finite = finite[np.isfinite(fv)]
    as32 = finite.view(np.float16).astype(np.float32)
    # every finite f16 survives f16 -> f32 -> f16
    back = np.array([L.kfo_f32_to_f16(float(v)) for v in as32], np.uint16)
    same = (back == finite) | ((finite & 0x7FFF) == 0)  # signed zeros compare by value below
    assert same.all()
    # midpoints between neighbouring f16 values (ties to even) and one f32 ulp either side of them
    pos = np.sort(np.unique(as32[(as32 > 0) & np.isfinite(as32)]))
    mids = ((pos[:-1].astype(np.float64) + pos[1:].astype(np.float64)) / 2).astype(np.float32)
    probes = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0)),
                             np.float32([65504.0, 65519.99, 65520.0, 1e9, 5.96e-8, 2.98e-8, 2.9802322e-08, 1e-30])])
    probes = np.concatenate([probes, -probes])
    rng = np.random.default_rng(7)
    probes = np.concatenate([probes, (rng.standard_normal(20000) * 10.0 ** rng.uniform(-9, 5, 20000)).astype(np.float32)])
    got = np.array([L.kfo_f32_to_f16(float(v)) for v in probes], np.uint16)
    want = probes.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ the reference's invariants

DOT_TYPES = [(12, [("f16", 0), ("f16", 2)]), (13, [("f16", 0), ("f16", 2)]), (14, [("f16", 208)]),
             (15, [("f32", 0)])]  # parity.rs:36-43, restricted to the restated types


def _patched_row(rng, ty, n, scales):
    block, size = oracle.LAYOUT[ty]
    src = np.array([rng.next() & 0xFF for _ in range(oracle.row_bytes(ty, n))], np.uint8)
    for b in range(n // block):
        blk = src[b * size : (b + 1) * size]
        for kind, at in scales:
            if kind == "f16":
                bits = (((5 + rng.next() % 8) << 10) | (rng.next() & 0x3FF)) & 0xFFFF
                blk[at : at + 2] = np.frombuffer(np.uint16(bits).tobytes(), np.uint8)
            else:
                v = np.float32(0.001 + 0.01 * rng.unit())
                blk[at : at + 4] = np.frombuffer(v.tobytes(), np.uint8)
    return src


def test_dot_row_matches_dequant_then_dot():
    """parity.rs:132-167, same seed and scale patching, for the K types; plus q8_0 with its f16 scale patched."""
    rng = SplitMix(0x6B66646F74726F77)
    for ty, scales in DOT_TYPES + [(8, [("f16", 0)])]:
        block, _ = oracle.LAYOUT[ty]
        n = 4 * block
        for _ in range(3):
            src = _patched_row(rng, ty, n, scales)
            x = np.array([2.0 * rng.unit() - 1.0 for _ in range(n)], np.float32)
            deq = oracle.dequant(ty, src, n)[0]
            want = float(np.dot(deq.astype(np.float64), x.astype(np.float64)))
            got = oracle.dot_row(ty, src, x)
            assert abs(got - want) / abs(want) <= 1e-3


@pytest.mark.parametrize("name,ty", [("q8_0", 8), ("q4_K", 12), ("q5_K", 13), ("q6_K", 14)])
def test_dot_i8_matches_dequant_then_dot(name, ty):
    """parity.rs:169-203 on the golden rows: err <= 1e-4 * sum|p| + 1e-6 against float64."""
    rng = SplitMix(0x6465717561_6E7474)
    n, rows_w, blocks, _ = oracle.load_fixture(os.path.join(GOLDEN, f"{name}.bin"))
    kind = oracle.act_kind(ty)
    rows = 3
    x = np.array([2.0 * rng.unit() - 1.0 for _ in range(rows * n)], np.float32).reshape(rows, n)
    q, d16, s16 = oracle.quantize_activations(kind, x)
    checked = 0
    for r in range(min(rows_w, 4)):
        deq = oracle.dequant(ty, blocks[r], n)[0].astype(np.float64)
        if not np.isfinite(deq).all():
            continue  # the fixtures' random scale bytes decode to inf/nan in some rows (bit-exact above all the same)
        checked += 1
        y = oracle.dot_i8(ty, blocks[r], q, d16, s16)
        for a in range(rows):
            xa = np.repeat(d16[a], 16).astype(np.float64) * q[a].astype(np.float64)
            p = deq * xa
            assert abs(float(y[a]) - p.sum()) <= 1e-4 * np.abs(p).sum() + 1e-6
    assert checked >= 1


# ------------------------------------------------------------------ integer block dots: brute force and special cases

def _q4k_decode(row, n):
    """q4_K bytes -> (d, dmin, sc[nsb][8], m[nsb][8], q[n] in 0..15) straight from the block definition."""
    nsb = n // 256
    blk = row.reshape(nsb, 144)
    d = blk[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float32)
    dmin = blk[:, 2:4].copy().view(np.float16)[:, 0].astype(np.float32)
    s = blk[:, 4:16].astype(np.int64)
    sc = np.zeros((nsb, 8), np.int64)
    m = np.zeros((nsb, 8), np.int64)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = blk[:, 16:].reshape(nsb, 4, 32).astype(np.int64)
    q = np.concatenate([qs & 0xF, qs >> 4], axis=2).reshape(nsb, 256)  # pair j: low nibbles then high nibbles
    return d, dmin, sc, m, q


def test_block_ints_q8_0_brute_force():
    rng = np.random.default_rng(1)
    n = 256
    w = rng.integers(0, 256, (4, oracle.row_bytes(8, n)), dtype=np.uint8)
    x = rng.standard_normal((2, n)).astype(np.float32)
    q, _, s16 = oracle.quantize_activations(3, x)
    for r in range(4):
        wq = w[r].reshape(-1, 34)[:, 2:].view(np.int8).astype(np.int64)
        for a in range(2):
            want = (wq * q[a].reshape(-1, 32).astype(np.int64)).sum(axis=1)
            assert np.array_equal(oracle.block_ints(8, w[r], q[a], s16[a]), want)


def test_block_ints_q4_k_brute_force_and_float_combine():
    rng = np.random.default_rng(2)
    n = 1024
    w = rng.integers(0, 256, (3, oracle.row_bytes(12, n)), dtype=np.uint8)
    w.reshape(3, -1, 144)[:, :, 0:2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
    w.reshape(3, -1, 144)[:, :, 2:4] = np.frombuffer(np.float16(0.003).tobytes(), np.uint8)
    x = rng.standard_normal((2, n)).astype(np.float32)
    q, d16, s16 = oracle.quantize_activations(4, x)
    for r in range(3):
        d, dmin, sc, m, wq = _q4k_decode(w[r], n)
        y = oracle.dot_i8(12, w[r], q, d16, s16)
        for a in range(2):
            qa = q[a].reshape(-1, 8, 32).astype(np.int64)
            dots = (wq.reshape(-1, 8, 32) * qa).sum(axis=2)
            sumi = (sc * dots).sum(axis=1)
            mins = (m * qa.sum(axis=2)).sum(axis=1)
            got = oracle.block_ints(12, w[r], q[a], s16[a]).reshape(-1, 2)
            assert np.array_equal(got[:, 0], sumi)
            assert np.array_equal(got[:, 1], mins)
            # the float combine of dot_i8 is d*dx*sumi - dmin*dx*mins per super-block
            dx = d16[a, ::16].astype(np.float64)
            want = (d * dx * sumi - dmin * dx * mins).sum()
            assert abs(float(y[a]) - want) <= 1e-5 * (np.abs(d * dx * sumi).sum() + np.abs(dmin * dx * mins).sum())


def test_q4_k_unit_scales_reduce_to_textbook_dot():
    """With every sub-block scale 1, every min 0 and d = 1, the q4_K integer dot is the plain dot of the nibbles."""
    rng = np.random.default_rng(3)
    n = 512
    nib = rng.integers(0, 16, n)
    row = np.zeros((n // 256, 144), np.uint8)
    row[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    row[:, 4:8] = 1  # sc 0..3 = 1, high bits of sc/m 4..7 = 0
    row[:, 8:12] = 0  # m 0..3 = 0
    row[:, 12:16] = 0x01  # sc 4..7 = 1, m 4..7 = 0
    for b in range(n // 256):
        for j in range(4):
            lo = nib[256 * b + 64 * j : 256 * b + 64 * j + 32]
            hi = nib[256 * b + 64 * j + 32 : 256 * b + 64 * j + 64]
            row[b, 16 + 32 * j : 48 + 32 * j] = lo | (hi << 4)
    row = row.ravel()
    x = rng.standard_normal((1, n)).astype(np.float32)
    q, d16, s16 = oracle.quantize_activations(4, x)
    got = oracle.block_ints(12, row, q[0], s16[0]).reshape(-1, 2)
    want = (nib.reshape(-1, 256) * q[0].reshape(-1, 256).astype(np.int64)).sum(axis=1)
    assert np.array_equal(got[:, 0], want)
    assert np.array_equal(got[:, 1], np.zeros_like(want))
    assert np.array_equal(oracle.dequant(12, row, n)[0], nib.astype(np.float32))


# ------------------------------------------------------------------ activation quantization: closed forms and ties

def test_quantize_activations_q8_0_closed_form():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((5, 256)) * rng.uniform(0.01, 30, (5, 1))).astype(np.float32)
    x[1, :32] = 0.0
    q, d16, s16 = oracle.quantize_activations(3, x)
    blk = x.reshape(5, -1, 32)
    amax = np.abs(blk).max(axis=2)
    d = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(np.repeat(d.astype(np.float16).astype(np.float32), 2, axis=1), d16)
    assert np.abs(q.astype(int)).max() <= 127
    assert (q.reshape(5, -1, 32)[1, 0] == 0).all() and d16[1, 0] == 0
    assert np.array_equal(s16, q.reshape(5, -1, 16).astype(np.int64).sum(axis=2))
    # reconstruction within half a step of the unrounded scale
    recon = q.reshape(5, -1, 32) * d[:, :, None]
    assert (np.abs(recon - blk) <= d[:, :, None] * 0.5001 + 1e-12).all()


def test_quantize_activations_rounding_ties():
    # Q8_0: amax 127 gives d = 1, so v * id = v and 2.5 rounds half away from zero to 3, -2.5 to -3
    x = np.zeros((1, 32), np.float32)
    x[0, :4] = [127.0, 2.5, -2.5, 0.5]
    q, d16, _ = oracle.quantize_activations(3, x)
    assert list(q[0, :4]) == [127, 3, -3, 1] and d16[0, 0] == 1.0
    # Q8K: max 127 gives iscale -1, so 2.5 -> -2.5 rounds half to even to -2, 3.5 -> -4
    x = np.zeros((1, 256), np.float32)
    x[0, :3] = [127.0, 2.5, 3.5]
    q, d16, _ = oracle.quantize_activations(4, x)
    assert list(q[0, :3]) == [-127, -2, -4] and d16[0, 0] == -1.0


def test_quantize_activations_hard_ties_round_the_f32_product():
    # v * id is exactly k + 0.5 in f32 while the real product is below it: the reference rounds the f32 product
    from tie_inputs import hard_tie_rows

    x, made = hard_tie_rows(2, 256, seed=1)
    assert made > 200
    q, _, _ = oracle.quantize_activations(3, x)
    b = x.reshape(2, -1, 32)
    idv = np.float32(1) / (np.abs(b).max(-1, keepdims=True) / np.float32(127)).astype(np.float32)
    p = (b * idv).astype(np.float32)
    want = (np.sign(p) * np.floor(np.abs(p) + np.float32(0.5))).astype(np.int8).reshape(2, -1)
    assert np.array_equal(q, want)


def test_quantize_activations_q8k_first_max_wins():
    x = np.zeros((2, 256), np.float32)
    x[0, 3], x[0, 10] = 5.0, -5.0   # +5 first: iscale = -127/5
    x[1, 3], x[1, 10] = -5.0, 5.0   # -5 first: iscale = +127/5
    q, d16, _ = oracle.quantize_activations(4, x)
    assert (q[0, 3], q[0, 10]) == (-127, 127) and d16[0, 0] < 0
    assert (q[1, 3], q[1, 10]) == (-127, 127) and d16[1, 0] > 0
    z = np.zeros((1, 256), np.float32)
    qz, dz, sz = oracle.quantize_activations(4, z)
    assert not qz.any() and not dz.any() and not sz.any()


def test_quantize_activations_rejects_bad_widths():
    assert oracle.quantize_activations(3, np.zeros((1, 48), np.float32)) is None
    assert oracle.quantize_activations(4, np.zeros((1, 128), np.float32)) is None
    assert oracle.quantize_activations(4, np.zeros((1, 40), np.float32)) is None


@pytest.mark.parametrize("kind", [3, 4])
def test_round_activations_equals_acti8_dequant(kind):
    """lib.rs:74-78 against :171-209: the floats round_activations multiplies are the dequantized int8 rows."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 512)).astype(np.float32) * 3
    q, d16, _ = oracle.quantize_activations(kind, x)
    for r in range(3):
        want = np.repeat(d16[r], 16) * q[r].astype(np.float32)
        assert np.array_equal(oracle.round_activations(kind, x[r]), want)


# ------------------------------------------------------------------ the CPU backend's product

@pytest.mark.parametrize("ty", [8, 12])
@pytest.mark.parametrize("rows", [1, 2, 3, 5])
def test_matmul_slice_against_float64(ty, rows):
    rng = np.random.default_rng(10 + rows)
    n_in, n_out = 512, 24
    w = np.stack([oracle.q8_0_quantize(rng.standard_normal(n_in).astype(np.float32) * 0.02)[0] for _ in range(n_out)]) if ty == 8 \
        else _random_q4k(rng, n_out, n_in)
    x = rng.standard_normal((rows, n_in)).astype(np.float32)
    bias = rng.standard_normal(n_out).astype(np.float32)
    y = oracle.matmul_slice(ty, w, n_in, n_out, x, bias)
    deq = oracle.dequant(ty, w, n_in).astype(np.float64)
    xr = np.stack([oracle.round_activations(oracle.act_kind(ty), x[r]) for r in range(rows)]).astype(np.float64)
    want = xr @ deq.T + bias
    mag = np.abs(xr) @ np.abs(deq).T + np.abs(bias)
    assert (np.abs(y - want) <= 1e-5 * mag + 1e-6).all()
    if rows <= 2:
        for r in range(rows):
            for o in range(0, n_out, 7):
                assert y[r, o] == np.float32(oracle.dot_row(ty, w[o], xr[r].astype(np.float32)) + bias[o])
    yi = oracle.matmul_i8(ty, w, n_in, n_out, x, bias)
    assert (np.abs(yi - want) <= 1e-4 * mag + 1e-6).all()


def _random_q4k(rng, rows, n):
    w = rng.integers(0, 256, (rows, n // 256, 144), dtype=np.uint8)
    w[:, :, 0:2] = np.frombuffer(np.float16(0.002).tobytes(), np.uint8)
    w[:, :, 2:4] = np.frombuffer(np.float16(0.001).tobytes(), np.uint8)
    return w.reshape(rows, -1)


def test_matmul_slice_rejects_bad_width():
    w = np.zeros((2, 34), np.uint8)
    with pytest.raises(AssertionError):
        oracle.matmul_slice(8, w, 48, 2, np.zeros((1, 48), np.float32))


def test_moe_ffn_composition():
    """moe::exec with selected experts equals the composition of its expert matvecs (float64 reference)."""
    rng = np.random.default_rng(6)
    n_exp, n_embd, n_ff, rows, used = 3, 256, 512, 4, 2
    gate = _random_q4k(rng, n_exp * n_ff, n_embd)
    up = _random_q4k(rng, n_exp * n_ff, n_embd)
    down = _random_q4k(rng, n_exp * n_embd, n_ff)
    x = rng.standard_normal((rows, n_embd)).astype(np.float32)
    sel = np.array([[0, 2], [1, -1], [2, 1], [-1, -1]], np.int32)
    wts = rng.uniform(0.1, 1, (rows, used)).astype(np.float32)
    out = oracle.moe_ffn(12, gate, up, down, n_exp, n_embd, n_ff, x, sel, wts)
    for r in range(rows):
        want = np.zeros(n_embd)
        for k in range(used):
            e = sel[r, k]
            if e < 0:
                continue
            xr = oracle.round_activations(4, x[r]).astype(np.float64)
            g = oracle.dequant(12, gate[e * n_ff : (e + 1) * n_ff], n_embd).astype(np.float64) @ xr
            u = oracle.dequant(12, up[e * n_ff : (e + 1) * n_ff], n_embd).astype(np.float64) @ xr
            h = (g / (1 + np.exp(-g))) * u
            hr = oracle.round_activations(4, h.astype(np.float32)).astype(np.float64)
            ye = oracle.dequant(12, down[e * n_embd : (e + 1) * n_embd], n_ff).astype(np.float64) @ hr
            want += wts[r, k] * ye
        scale = np.abs(want).max() + 1e-3
        assert np.abs(out[r] - want).max() <= 2e-3 * scale, r
    assert not out[3].any()


def test_moe_ffn_i8_is_the_int8_composition_and_near_the_float_path():
    """experts::hidden_rows + down_cols: per pair, gate/up by matmul_i8, silu(g) * u, down by matmul_i8 on the hidden
    row, weighted in selection order; and within the reference's own int8-vs-float bound of the float path
    (crates/kf-backend-cpu/src/experts.rs:181-217: 2e-2 of the mean magnitude)."""
    rng = np.random.default_rng(8)
    n_exp, n_embd, n_ff, rows, used = 3, 256, 512, 4, 2
    gate = _random_q4k(rng, n_exp * n_ff, n_embd)
    up = _random_q4k(rng, n_exp * n_ff, n_embd)
    down = _random_q4k(rng, n_exp * n_embd, n_ff)
    x = rng.standard_normal((rows, n_embd)).astype(np.float32)
    sel = np.array([[0, 2], [1, -1], [2, 1], [-1, -1]], np.int32)
    wts = rng.uniform(0.1, 1, (rows, used)).astype(np.float32)
    out = oracle.moe_ffn_i8(12, gate, up, down, n_exp, n_embd, n_ff, x, sel, wts)
    for r in range(rows):
        want = np.zeros(n_embd, np.float32)
        for k in range(used):
            e = sel[r, k]
            if e < 0:
                continue
            g = oracle.matmul_i8(12, gate[e * n_ff : (e + 1) * n_ff], n_embd, n_ff, x[r])[0]
            u = oracle.matmul_i8(12, up[e * n_ff : (e + 1) * n_ff], n_embd, n_ff, x[r])[0]
            h = np.array([oracle.silu(float(v)) for v in g], np.float32) * u
            y = oracle.matmul_i8(12, down[e * n_embd : (e + 1) * n_embd], n_ff, n_embd, h)[0]
            want = want + wts[r, k] * y
        assert np.array_equal(out[r], want), r
    flt = oracle.moe_ffn(12, gate, up, down, n_exp, n_embd, n_ff, x, sel, wts)
    live = np.abs(flt[:3]).mean()
    assert np.abs(out - flt).max() <= 2e-2 * live
    assert not out[3].any()


def _q5k_decode(row, n):
    """q5_K bytes -> (d, dmin, sc, m, q[n] in 0..31): q4_K's header and nibbles, the fifth bit of element l of
    sub-block s from bit s of qh[l] (the block definition, crates/kf-quant/src/types/q5_k.rs:67-93)."""
    nsb = n // 256
    blk = row.reshape(nsb, 176)
    as_q4k = np.concatenate([blk[:, :16], blk[:, 48:]], axis=1)
    d, dmin, sc, m, q4 = _q4k_decode(as_q4k.ravel(), n)
    qh = blk[:, 16:48].astype(np.int64)                     # [nsb][32]
    hb = np.stack([(qh >> s) & 1 for s in range(8)], axis=1)  # [nsb][8][32]
    return d, dmin, sc, m, q4 + 16 * hb.reshape(nsb, 256)


def _q6k_decode(row, n):
    """q6_K bytes -> (d, sc[nsb][16] int8, q[n] in -32..31) by the element map of quads (q6_k.rs:7-15)."""
    nsb = n // 256
    blk = row.reshape(nsb, 210)
    d = blk[:, 208:210].copy().view(np.float16)[:, 0].astype(np.float32)
    sc = blk[:, 192:208].view(np.int8).astype(np.int64)
    q = np.zeros((nsb, 256), np.int64)
    for h in range(2):
        ql = blk[:, 64 * h : 64 * h + 64].astype(np.int64)
        qh = blk[:, 128 + 32 * h : 160 + 32 * h].astype(np.int64)
        l = np.arange(32)
        q[:, 128 * h + l] = (ql[:, l] & 0xF) | ((qh[:, l] & 3) << 4)
        q[:, 128 * h + 32 + l] = (ql[:, l + 32] & 0xF) | (((qh[:, l] >> 2) & 3) << 4)
        q[:, 128 * h + 64 + l] = (ql[:, l] >> 4) | (((qh[:, l] >> 4) & 3) << 4)
        q[:, 128 * h + 96 + l] = (ql[:, l + 32] >> 4) | (((qh[:, l] >> 6) & 3) << 4)
    return d, sc, q - 32


@pytest.mark.parametrize("name,ty", [("q5_K", 13), ("q6_K", 14)])
def test_numpy_decoders_reproduce_ggml_dequant(name, ty):
    """The brute-force decoders below are themselves pinned to ggml's fixtures (element map and scales)."""
    n, rows, blocks, want = oracle.load_fixture(os.path.join(GOLDEN, f"{name}.bin"))
    for r in range(rows):
        if ty == 13:
            d, dmin, sc, m, q = _q5k_decode(blocks[r], n)
            deq = (d[:, None, None] * sc[:, :, None]) * q.reshape(-1, 8, 32) - (dmin[:, None, None] * m[:, :, None])
        else:
            d, sc, q = _q6k_decode(blocks[r], n)
            deq = (d[:, None, None] * sc[:, :, None]) * q.reshape(-1, 16, 16)
        assert np.allclose(deq.reshape(-1), want[r], rtol=1e-6, atol=1e-6, equal_nan=True)


def test_block_ints_q5_k_and_q6_k_brute_force():
    rng = np.random.default_rng(4)
    n = 1024
    x = rng.standard_normal((2, n)).astype(np.float32)
    q, d16, s16 = oracle.quantize_activations(4, x)
    for ty in (13, 14):
        w = rng.integers(0, 256, (3, oracle.row_bytes(ty, n)), dtype=np.uint8)
        for r in range(3):
            for a in range(2):
                got = oracle.block_ints(ty, w[r], q[a], s16[a])
                qa = q[a].astype(np.int64)
                if ty == 13:
                    _, _, sc, m, wq = _q5k_decode(w[r], n)
                    dots = (wq.reshape(-1, 8, 32) * qa.reshape(-1, 8, 32)).sum(axis=2)
                    bsum = s16[a].reshape(-1, 8, 2).sum(axis=2).astype(np.int64)
                    want = np.stack([(sc * dots).sum(axis=1), (m * bsum).sum(axis=1)], axis=1).ravel()
                else:
                    _, sc, wq = _q6k_decode(w[r], n)
                    # the signed values' group dots, which the integer form reaches as (q + 32) . x - 32 sum16
                    dots = (wq.reshape(-1, 16, 16) * qa.reshape(-1, 16, 16)).sum(axis=2)
                    assert np.array_equal(dots, ((wq + 32).reshape(-1, 16, 16) * qa.reshape(-1, 16, 16)).sum(axis=2)
                                          - 32 * s16[a].reshape(-1, 16).astype(np.int64))
                    want = (sc * dots).sum(axis=1)
                assert np.array_equal(got, want), (ty, r, a)
