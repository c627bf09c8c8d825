"""Pins for the CPU oracle (runs on CPU).

Each oracle function is checked against something other than its own formula:
golden vectors written by the reference (tests/golden/make_golden.py), closed
forms, float64 brute force, and invariants chosen so that a plausible slip (a
dropped zero point, a transposed operand, single-rounding `x/s+z`, round-half-up)
fails at least one of them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import paged as op
from oracle import quant as oq
from oracle import tree as ot
from tests._helpers import assert_quant_equal, golden_cache, golden_quant, load_npz

F32 = np.float32


# ---- quantizer -------------------------------------------------------------------------------

def test_quantize_matches_reference_golden_vectors():
    d = load_npz("quant_golden.npz")
    for name in d["names"]:
        x = d[f"{name}_x"]
        ref = golden_quant(d, name)
        mine = oq.quantize_int8_per_block(x, ref.block_size)
        assert mine.original_shape == ref.original_shape
        assert_quant_equal(mine, ref, name)
        deq = oq.dequantize_int8_per_block(mine)
        assert np.array_equal(deq.view(np.uint32), d[f"{name}_deq"].view(np.uint32)), name


def test_quantize_closed_forms():
    # all-zero block -> uint8 0 (int8 -128), scale = fp32(1e-8), zero 0; round-trips to exact 0
    q = oq.quantize_int8_per_block(np.zeros((1, 1, 16, 8), F32), 16)
    assert (q.values == -128).all() and q.zero_point.item() == 0
    assert q.scale.item() == F32(1e-8)
    assert (oq.dequantize_int8_per_block(q) == 0).all()
    # constant positive block: min = max = c > 0 -> scale floor, zero clamps to 0, codes clamp to 255
    q = oq.quantize_int8_per_block(np.full((1, 1, 16, 4), 3.0, F32), 16)
    assert q.scale.item() == F32(1e-8) and q.zero_point.item() == 0 and (q.values == 127).all()
    # a block spanning [-1, 1]: scale = fl(2/255), zero = rint(fl(1/scale)); the minimum lands on
    # code 0 (|mn/s + zero| <= 1/2) and the maximum on 254 or 255 (255 + zero - (-mn/s) rounded)
    x = np.linspace(-1.0, 1.0, 16 * 4, dtype=F32).reshape(1, 1, 16, 4)
    q = oq.quantize_int8_per_block(x, 16)
    s = F32(2.0) / F32(255.0)
    assert q.scale.item() == s
    assert q.zero_point.item() == int(np.rint(F32(1.0) / s))
    u = q.values.astype(np.int16) + 128
    assert u.min() == 0 and u.max() in (254, 255)
    # codes increase monotonically with x inside a block
    assert (np.diff(u.ravel()) >= 0).all()


def test_quantize_codes_are_nearest_with_two_roundings():
    """Brute force: each code is the half-even nearest integer of fl(fl(x/s) + z), clamped."""

    rng = np.random.default_rng(3)
    x = (rng.standard_normal((3, 2, 40, 24)) * rng.uniform(0.1, 5, (3, 2, 1, 1))).astype(F32)
    q = oq.quantize_int8_per_block(x, 16)
    u = q.values.astype(np.int64) + 128
    xp = np.pad(x, ((0, 0), (0, 0), (0, 8), (0, 0)))  # 40 -> 48 rows
    for idx in np.ndindex(3, 2, 3):
        blk = xp[idx[0], idx[1], idx[2] * 16:(idx[2] + 1) * 16]
        s = q.scale[idx[0], idx[1], idx[2], 0, 0]
        z = float(q.zero_point[idx[0], idx[1], idx[2], 0, 0])
        assert s == max(F32((F32(blk.max()) - F32(blk.min()))) / F32(255.0), F32(1e-8))
        t = (blk / s).astype(F32) + F32(z)  # two roundings
        for val, code in zip(t.ravel()[::7], u[idx[0], idx[1], idx[2]].ravel()[::7]):
            lo = math.floor(val)
            frac = float(val) - lo
            want = lo + 1 if frac > 0.5 or (frac == 0.5 and lo % 2 == 1) else lo
            assert code == min(max(want, 0), 255)


def test_symmetric_per_token_closed_forms():
    """Symmetric absmax INT8 per token: the extreme of each row maps to +-127, zero rows keep
    the 1e-8 floor, negation negates the codes, and the layout reads back through the affine
    dequantizer as q * scale."""

    x = np.array([[[[0.5, -2.0, 1.0, 0.0], [0.0, 0.0, 0.0, 0.0], [3.0, 3.0, -3.0, 1.5]]]], F32)
    q = oq.quantize_int8_symmetric_per_token(x)
    assert q.block_size == 1 and q.values.shape == (1, 1, 3, 1, 4) and (q.zero_point == 128).all()
    s = q.scale.reshape(3)
    assert s[0] == F32(2.0) / F32(127.0) and s[1] == F32(1e-8) and s[2] == F32(3.0) / F32(127.0)
    codes = q.values.reshape(3, 4).astype(np.int64)
    assert codes[0, 1] == -127 and codes[2, 0] == 127 and codes[2, 2] == -127
    assert (codes[1] == 0).all()
    qn = oq.quantize_int8_symmetric_per_token(-x)
    assert (qn.values.astype(np.int64) == -q.values.astype(np.int64)).all()
    deq = oq.dequantize_int8_per_block(q)
    assert np.array_equal(deq.reshape(3, 4), (codes.astype(F32) * s[:, None]).astype(F32))


def test_symmetric_per_token_codes_are_nearest():
    """Brute force: every code is the half-even nearest integer of fl(x / s), |code| <= 127."""

    rng = np.random.default_rng(9)
    x = (rng.standard_normal((2, 3, 17, 24)) * rng.uniform(0.01, 50, (2, 3, 17, 1))).astype(F32)
    q = oq.quantize_int8_symmetric_per_token(x)
    s = q.scale.reshape(2, 3, 17, 1)
    assert np.array_equal(s, np.maximum(np.abs(x).max(-1, keepdims=True) / F32(127.0), F32(1e-8)))
    t = (x / s).astype(F32)
    codes = q.values.reshape(2, 3, 17, 24).astype(np.int64)
    for val, code in zip(t.ravel()[::5], codes.ravel()[::5]):
        lo = math.floor(val)
        frac = float(val) - lo
        want = lo + 1 if frac > 0.5 or (frac == 0.5 and lo % 2 == 1) else lo
        assert code == min(max(want, -127), 127)


def test_dequantize_error_bound_and_padding_crop():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 3, 19, 16)).astype(F32)
    q = oq.quantize_int8_per_block(x, 8)
    y = oq.dequantize_int8_per_block(q)
    assert y.shape == x.shape
    half_step = np.repeat(q.scale.reshape(2, 3, 3), 8, axis=-1)[..., :19, None] * 0.5 + 1e-6
    assert (np.abs(x - y) <= half_step).all()
    assert np.abs(x - y).max() < 0.03  # the reference's own bound (test_flashspec.py:36-41)


# ---- attention -------------------------------------------------------------------------------

@pytest.mark.parametrize("lengths", [None, [5, 2, 0]])
def test_reference_attention_matches_float64_brute_force(lengths):
    rng = np.random.default_rng(11)
    q = rng.standard_normal((3, 2, 8)).astype(F32)
    k = rng.standard_normal((3, 2, 5, 8)).astype(F32)
    v = rng.standard_normal((3, 2, 5, 8)).astype(F32)
    lens = None if lengths is None else np.asarray(lengths)
    got = oa.reference_attention(q, k, v, lens)
    want = oa.reference_attention_f64_loops(q, k, v, lens)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_attention_closed_forms():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((2, 3, 16)).astype(F32)
    v = rng.standard_normal((2, 3, 7, 16)).astype(F32)
    # one valid token -> that token's V
    k = rng.standard_normal((2, 3, 7, 16)).astype(F32)
    out = oa.reference_attention(q, k, v, np.asarray([1, 1]))
    np.testing.assert_allclose(out, v[:, :, 0, :], rtol=1e-6, atol=1e-6)
    # identical keys -> uniform weights -> mean of V
    k_same = np.repeat(k[:, :, :1, :], 7, axis=2)
    np.testing.assert_allclose(oa.reference_attention(q, k_same, v), v.mean(axis=2), rtol=1e-5, atol=1e-6)
    # masking == truncation
    lens = np.asarray([4, 6])
    masked = oa.reference_attention(q, k, v, lens)
    for b, L in enumerate(lens):
        trunc = oa.reference_attention(q[b:b + 1], k[b:b + 1, :, :L], v[b:b + 1, :, :L])
        np.testing.assert_allclose(masked[b:b + 1], trunc, rtol=1e-6, atol=1e-6)
    # zero-length row averages V uniformly (attention.py:109-117 semantics)
    z = oa.reference_attention(q, k, v, np.asarray([0, 7]))
    np.testing.assert_allclose(z[0], v[0].mean(axis=1), rtol=1e-5, atol=1e-6)


def test_fused_oracle_equals_dense_attention_on_dequantized_kv():
    rng = np.random.default_rng(8)
    q = rng.standard_normal((2, 3, 16)).astype(F32)
    k = rng.standard_normal((2, 3, 25, 16)).astype(F32)
    v = rng.standard_normal((2, 3, 25, 16)).astype(F32)
    kq, vq = oq.quantize_int8_per_block(k, 8), oq.quantize_int8_per_block(v, 8)
    got = oa.fused_dequant_attention(q, kq, vq)
    want = oa.reference_attention_f64_loops(q, oq.dequantize_int8_per_block(kq), oq.dequantize_int8_per_block(vq))
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


# ---- paged layout, append, allocator --------------------------------------------------------

def test_layouts_match_reference_golden_tables_and_stores():
    d = load_npz("layout_golden.npz")
    k, v, lengths = d["k"], d["v"], d["lengths"]
    for key in ("contiguous0", "shuffled13", "shuffled0", "interleaved0"):
        ref = golden_cache(d, key)
        table = ref.block_table
        perm = None
        if key != "contiguous0":
            perm = np.empty(table.size, dtype=np.int64)
            perm[table.ravel()] = np.arange(table.size)
        mine = op.from_dense(k, v, 4, lengths=lengths, perm=perm)
        assert np.array_equal(mine.block_table, table), key
        assert_quant_equal(mine.k_quant, ref.k_quant, key + "/k")
        assert_quant_equal(mine.v_quant, ref.v_quant, key + "/v")
    ref = golden_cache(d, "interleaved0")
    inter = op.interleaved_perm(3, 5)  # closed form of paged.py:392-393
    inv = np.empty_like(inter)
    inv[inter] = np.arange(inter.size)
    assert np.array_equal(inv.reshape(3, 5), ref.block_table)


def test_layouts_preserve_logical_kv():
    rng = np.random.default_rng(4)
    k = rng.standard_normal((3, 2, 17, 8)).astype(F32)
    v = rng.standard_normal((3, 2, 17, 8)).astype(F32)
    base = op.to_dense(op.from_dense(k, v, 4))
    for perm in (op.interleaved_perm(3, 5), rng.permutation(15)):
        other = op.to_dense(op.from_dense(k, v, 4, perm=perm))
        assert np.array_equal(base[0], other[0]) and np.array_equal(base[1], other[1])
    assert np.abs(base[0] - k).max() < 0.03


def test_append_matches_reference_golden_vectors():
    d = load_npz("append_golden.npz")
    for name in d["names"]:
        cin, cout = golden_cache(d, f"{name}_in"), golden_cache(d, f"{name}_out")
        mine = op.append(cin, d[f"{name}_kn"], d[f"{name}_vn"])
        assert np.array_equal(mine.block_table, cout.block_table), name
        assert np.array_equal(mine.lengths, cout.lengths), name
        assert mine.max_seq_len == cout.max_seq_len
        assert_quant_equal(mine.k_quant, cout.k_quant, f"{name}/k")
        assert_quant_equal(mine.v_quant, cout.v_quant, f"{name}/v")
        att = oa.paged_quant_attention(d[f"{name}_q"], mine)
        np.testing.assert_allclose(att, d[f"{name}_attn"], rtol=1e-5, atol=1e-5)


def replay_allocator_script(d):
    H, D, bs, cap = (int(x) for x in d["config"])
    alloc = op.OracleAllocator(cap, H, D, bs)
    for step, (op_code, rid, _n) in enumerate(d["script"]):
        if op_code == 0:
            alloc.add_request(int(rid), d[f"s{step}_k"], d[f"s{step}_v"])
        elif op_code == 1:
            alloc.append_request(int(rid), d[f"s{step}_k"], d[f"s{step}_v"])
        else:
            alloc.release_request(int(rid))
        yield step, alloc


def test_allocator_lifecycle_matches_reference_golden_vectors():
    d = load_npz("allocator_golden.npz")
    for step, alloc in replay_allocator_script(d):
        assert np.array_equal(alloc.k_quant.values, d[f"s{step}_kvalues"]), step
        assert np.array_equal(alloc.k_quant.scale.view(np.uint32), d[f"s{step}_kscale"].view(np.uint32)), step
        assert np.array_equal(alloc.k_quant.zero_point, d[f"s{step}_kzero"]), step
        assert np.array_equal(alloc.v_quant.values, d[f"s{step}_vvalues"]), step
        live = list(alloc.requests)
        assert live == d[f"s{step}_live"].tolist()
        if live:
            c = alloc.to_cache(live)
            assert np.array_equal(c.block_table, d[f"s{step}_table"]), step
            assert np.array_equal(c.lengths, d[f"s{step}_lengths"]), step
        assert cap_allocated(alloc) == float(d[f"s{step}_allocated"])


def cap_allocated(alloc) -> float:
    return float(alloc.capacity_blocks - len(alloc.free))


def test_allocator_reuses_lowest_released_page():
    alloc = op.OracleAllocator(6, 2, 8, 4)
    rng = np.random.default_rng(0)
    alloc.add_request(10, rng.standard_normal((1, 2, 5, 8)).astype(F32), rng.standard_normal((1, 2, 5, 8)).astype(F32))
    alloc.add_request(20, rng.standard_normal((1, 2, 3, 8)).astype(F32), rng.standard_normal((1, 2, 3, 8)).astype(F32))
    released = alloc.requests[20]["blocks"][0]
    alloc.release_request(20)
    alloc.add_request(30, np.zeros((1, 2, 1, 8), F32), np.zeros((1, 2, 1, 8), F32))
    assert alloc.requests[30]["blocks"][0] == released == 2


# ---- tree verification -------------------------------------------------------------------------

def _tree_case(B, H, S, D, N, seed, lengths):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((B, H, S, D)).astype(F32)
    v = rng.standard_normal((B, H, S, D)).astype(F32)
    cache = op.from_dense(k, v, 4, lengths=np.asarray(lengths, dtype=np.int64))
    q = rng.standard_normal((B, N, H, D)).astype(F32)
    dk = rng.standard_normal((B, N, H, D)).astype(F32)
    dv = rng.standard_normal((B, N, H, D)).astype(F32)
    return q, cache, dk, dv


def test_tree_mask_formulation_matches_f64_parent_walk():
    q, cache, dk, dv = _tree_case(2, 2, 13, 8, 6, 1, [13, 5])
    parents = np.array([[-1, 0, 0, 1, 3, -1], [-1, -1, 1, 2, 0, 4]])
    got = ot.tree_verify_attention(q, cache, dk, dv, parents)
    ref = ot.tree_verify_f64_loops(q, cache, dk, dv, parents)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)


def test_tree_chain_and_star_equal_attention_on_concatenated_kv():
    """Chain: node n sees prefix + draft[0..n]; star: prefix + draft[n] only.  Both against
    reference_attention on explicitly concatenated K/V (a formulation without any mask)."""

    B, H, S, D, N = 2, 3, 11, 8, 4
    q, cache, dk, dv = _tree_case(B, H, S, D, N, 2, [11, 7])
    kp, vp = op.to_dense(cache)
    chain = np.array([[-1, 0, 1, 2]] * B)
    star = np.array([[-1, -1, -1, -1]] * B)
    got_chain = ot.tree_verify_attention(q, cache, dk, dv, chain)
    got_star = ot.tree_verify_attention(q, cache, dk, dv, star)
    for b in range(B):
        L = int(cache.lengths[b])
        for n in range(N):
            for sel, got in (([*range(n + 1)], got_chain), ([n], got_star)):
                keys = np.concatenate([kp[b:b + 1, :, :L], dk[b:b + 1, sel].transpose(0, 2, 1, 3)], axis=2)
                vals = np.concatenate([vp[b:b + 1, :, :L], dv[b:b + 1, sel].transpose(0, 2, 1, 3)], axis=2)
                ref = oa.reference_attention(q[b:b + 1, n], keys, vals)
                np.testing.assert_allclose(got[b:b + 1, n], ref, rtol=2e-5, atol=2e-6)


def test_tree_rejects_malformed_parents():
    for bad in ([[0, -1]], [[-1, 1]], [[-1, 2, 0]], [[-2, -1]]):
        with pytest.raises(ValueError):
            ot.validate_parents(np.array(bad))
    assert ot.path_mask(np.array([[-1, 0, 0, 2]]))[0].tolist() == [
        [True, False, False, False], [True, True, False, False], [True, False, True, False],
        [True, False, True, True]]


# ---- FP8 E4M3 per-block format (oracle/fp8.py): pinned against torch's float8_e4m3fn -------

def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_fp8_table_matches_torch():
    from oracle import fp8

    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    tab = fp8.e4m3_table()
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(tab), ~fin)
    assert np.array_equal(tab[fin], ref[fin].astype(np.float64))
    assert tab[0x7E] == 448.0 and tab[0x01] == 2.0 ** -9 and tab[0x08] == 2.0 ** -6


def test_fp8_encoder_matches_torch_on_codes_ties_and_random():
    from oracle import fp8

    tab = fp8.e4m3_table()
    pos = np.unique(np.abs(tab[np.isfinite(tab)]))
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)  # every rounding tie (exact in fp32)
    rng = np.random.default_rng(3)
    xs = np.concatenate([pos, -pos, mids, -mids, np.nextafter(mids, np.float32(np.inf)),
                         np.nextafter(mids, np.float32(0)), rng.uniform(-448, 448, 20000),
                         rng.standard_normal(20000) * 2.0 ** -8, [0.0, -0.0, 448.0, -448.0]]).astype(np.float32)
    xs = xs[np.abs(xs) <= 448]
    assert np.array_equal(fp8.encode_e4m3_rne(xs), _torch_e4m3(xs))
    with pytest.raises(ValueError):
        fp8.encode_e4m3_rne(np.array([449.0], dtype=np.float32))


def test_fp8_block_quantizer_closed_forms():
    from oracle import fp8

    rng = np.random.default_rng(4)
    x = (rng.standard_normal((2, 3, 37, 24)) * np.array([1.0, 1e-3, 50.0])[None, :, None, None]).astype(np.float32)
    q = fp8.quantize_fp8_per_block(x, 16)
    assert q.values.dtype == np.uint8 and q.values.shape == (2, 3, 3, 16, 24)
    assert q.scale.shape == (2, 3, 3, 1, 1) and not q.zero_point.any()
    # scale = max(absmax / 448, 1e-8) in float32; the block maximum becomes the extreme code
    blocks = oq.pad_sequence_dim(x, 16).reshape(2, 3, 3, 16, 24)
    amax = np.abs(blocks).max(axis=(-2, -1), keepdims=True)
    assert np.array_equal(q.scale, np.maximum(amax / np.float32(448), np.float32(1e-8)).astype(np.float32))
    flat_v = q.values.reshape(2, 3, 3, -1)
    flat_x = blocks.reshape(2, 3, 3, -1)
    arg = np.abs(flat_x).argmax(axis=-1)
    ext = np.take_along_axis(flat_v, arg[..., None], axis=-1)[..., 0]
    assert set(np.unique(ext & 0x7F)) == {0x7E}
    # brute force: every code is the nearest representable value to x / scale (ties even)
    tab = fp8.e4m3_table()
    y = np.clip(blocks / q.scale, -448, 448).astype(np.float32)
    got = tab[q.values].astype(np.float64)
    fin = tab[np.isfinite(tab)]
    best = np.abs(y[..., None].astype(np.float64) - fin).min(axis=-1)
    assert np.array_equal(np.abs(got - y.astype(np.float64)), best)
    # error bound of a 3-bit mantissa: half an ulp, relative 2^-4 in the normal range
    back = fp8.dequantize_fp8_per_block(q)
    normal = np.abs(x / q.scale.repeat(16, axis=-3).reshape(2, 3, 48, 1)[:, :, :37]) >= 2.0 ** -6
    rel = np.abs(back - x)[normal] / np.abs(x)[normal]
    assert rel.max() <= 2.0 ** -4 * (1 + 1e-6)


def test_fp8_zero_block_and_padding():
    from oracle import fp8

    x = np.zeros((1, 20, 8), dtype=np.float32)
    x[0, 3, 2] = -1.5
    q = fp8.quantize_fp8_per_block(x, 16)
    assert q.scale[0, 1, 0, 0] == np.float32(1e-8)   # all-zero second block (incl. padding)
    assert not q.values[0, 1].any()
    assert q.values[0, 0, 3, 2] == 0xFE               # -448: the block's extreme, negative
    back = fp8.dequantize_fp8_per_block(q)
    assert back.shape == x.shape and back[0, 3, 2] == np.float32(-1.5)
    assert np.array_equal(back[0, 4:], x[0, 4:])


# ---- per-channel affine INT8 (quant.quantize_int8_per_channel) -------------------------------

def test_per_channel_equals_per_block_on_each_column():
    """Each channel column of a block is the reference's per-block quantizer on that column
    (which the reference's golden vectors pin), padding and all."""

    rng = np.random.default_rng(8)
    x = (rng.standard_normal((2, 3, 45, 12)) * rng.uniform(0.01, 30, size=12)).astype(np.float32)
    pc = oq.quantize_int8_per_channel(x, 16)
    assert pc.values.shape == (2, 3, 3, 16, 12) and pc.scale.shape == (2, 3, 3, 1, 12)
    for d in range(12):
        col = oq.quantize_int8_per_block(x[..., d:d + 1], 16)
        assert np.array_equal(pc.values[..., d:d + 1], col.values)
        assert np.array_equal(pc.scale[..., d:d + 1], col.scale)
        assert np.array_equal(pc.zero_point[..., d:d + 1], col.zero_point)
    back = oq.dequantize_int8_per_block(pc)
    assert back.shape == x.shape
    assert np.abs(back - x).max() <= 0.5 * pc.scale.max() * (1 + 1e-5)
    # the generic dequantize dispatch reads it as the affine format
    assert np.array_equal(oq.dequantize(pc), back)
