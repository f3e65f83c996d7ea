"""Pin the oracle before trusting it: known answers, a brute force, a library routine, invariants.

Each check is chosen so that a plausible mistake in the oracle fails it: a
dropped scale or wrong GQA index fails the brute force and SDPA comparisons, a
missed mask fails the NaN-poisoned cases, a wrong slot formula fails the known
answers restated from the reference's tests.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import paged
from oracle.numerics import bits_to_f32, e4m3_to_f32, f32_to_bits, f32_to_e4m3, half_ulp, parity_report
from tests._support import build_scenario, brute_force

GOLDEN = Path(__file__).resolve().parent / "golden"
KNOWN = json.loads((GOLDEN / "known_answers.json").read_text())


# --- conversions ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype,torch_dtype", [("bf16", torch.bfloat16), ("fp16", torch.float16)])
def test_widening_matches_torch_for_every_bit_pattern(dtype: str, torch_dtype: torch.dtype) -> None:
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = bits_to_f32(bits, dtype)
    theirs = torch.from_numpy(bits.view(np.int16)).view(torch_dtype).float().numpy()
    both_nan = np.isnan(ours) & np.isnan(theirs)
    assert np.array_equal(ours[~both_nan], theirs[~both_nan])
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))


@pytest.mark.parametrize("dtype,torch_dtype", [("bf16", torch.bfloat16), ("fp16", torch.float16)])
def test_rounding_matches_torch(dtype: str, torch_dtype: torch.dtype) -> None:
    rng = np.random.default_rng(7)
    raw = rng.integers(0, 1 << 32, size=200_000, dtype=np.uint64).astype(np.uint32)
    values = raw.view(np.float32)
    # halfway cases of bf16 and fp16, signed zeros, infinities, denormals
    special = np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 65504.0, 65520.0, 1.0 + 2**-8,
                        1.0 + 3 * 2**-8, 1.0 + 2**-11, 1.0 + 3 * 2**-11], dtype=np.float32)
    values = np.concatenate([values, special])
    ours = f32_to_bits(values, dtype)
    theirs = torch.from_numpy(values).to(torch_dtype).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(values)
    assert np.array_equal(ours[~nan], theirs[~nan])
    assert np.isnan(bits_to_f32(ours[nan], dtype)).all()


def test_e4m3_decoding_matches_torch_for_every_code() -> None:
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = e4m3_to_f32(codes)
    assert np.array_equal(np.isnan(want), np.isnan(got))
    assert np.array_equal(want[~np.isnan(want)], got[~np.isnan(got)])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6 and np.isnan(got[0xFF])


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_e4m3_encoding_matches_torch_for_every_16_bit_input(dtype: str) -> None:
    # every bf16 / fp16 value a KV write can receive, NaN and infinities included
    values = bits_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16), dtype)
    want = torch.from_numpy(values).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(f32_to_e4m3(values), want)


def test_e4m3_encoding_matches_torch_on_float32_and_the_rounding_edges() -> None:
    rng = np.random.default_rng(5)
    values = (rng.standard_normal(200_000) * np.exp2(rng.uniform(-14, 10, 200_000))).astype(np.float32)
    edges = np.array([448.0, 464.0, np.nextafter(464.0, 500.0), 479.9, 480.0, 1e30, 0.0, -0.0,
                      2.0 ** -10, 1.5 * 2.0 ** -9, 2.5 * 2.0 ** -9, 2.0 ** -6, 2.0 ** -6 - 2.0 ** -10,
                      np.inf, -np.inf, np.nan], dtype=np.float32)
    values = np.concatenate([values, edges, -edges])
    want = torch.from_numpy(values).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(f32_to_e4m3(values), want)
    # ties go to the even code: 464 is halfway between 448 (0x7E) and the NaN code, 2.5 * 2^-9 between 2 and 3
    assert f32_to_e4m3(np.array([464.0, 1.5 * 2.0 ** -9, 2.5 * 2.0 ** -9], np.float32)).tolist() == [0x7E, 2, 2]
    # decoding what was encoded returns the value wherever it is representable
    finite = e4m3_to_f32(np.arange(256, dtype=np.uint8))
    finite = finite[~np.isnan(finite)]
    assert np.array_equal(e4m3_to_f32(f32_to_e4m3(finite)), finite)


def test_scaled_e4m3_encoding_matches_torch() -> None:
    # codes of float32(x) * float32(1 / scale), as torch's cast of that float32 product gives
    # them; scale 1 is the unscaled encoder; a power-of-two scale shifts the code's exponent only
    from oracle.numerics import f32_to_e4m3_scaled

    rng = np.random.default_rng(9)
    x = (rng.standard_normal(50_000) * np.exp2(rng.uniform(-12, 13, 50_000))).astype(np.float32)
    for scale in (1.0, 8.928571, 0.37, 4096.0, 2.0 ** -5):
        inverse = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(scale, dtype=torch.float32)
        want = (torch.from_numpy(x) * inverse).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        got = f32_to_e4m3_scaled(x, scale)
        assert np.array_equal(got, want), scale
    assert np.array_equal(f32_to_e4m3_scaled(x, 1.0), f32_to_e4m3(x))
    small = x[np.abs(x) < 100]
    shifted = e4m3_to_f32(f32_to_e4m3_scaled(small, 4.0)) * 4.0
    plain = e4m3_to_f32(f32_to_e4m3(small))
    normal = np.abs(small) >= 4 * 2.0 ** -6  # away from the subnormal range of either encoding
    assert np.array_equal(shifted[normal], plain[normal])


def test_scaled_codec_is_the_fp8_codec_with_scales() -> None:
    import pickle

    from ayaka_amd.kvcache import FP8_E4M3_CODEC, codec_scales, fp8_e4m3_codec

    codec = fp8_e4m3_codec(k_scale=4000 / 448, v_scale=0.1)
    assert codec == FP8_E4M3_CODEC and hash(codec) == hash(FP8_E4M3_CODEC)
    assert {FP8_E4M3_CODEC: 1}[codec] == 1
    k_scale, v_scale = codec_scales(codec)
    assert k_scale == float(np.float32(4000 / 448)) and v_scale == float(np.float32(0.1))  # float32, as read
    assert codec_scales(FP8_E4M3_CODEC) == (1.0, 1.0) and codec_scales("raw") == (1.0, 1.0)
    assert codec_scales(pickle.loads(pickle.dumps(codec))) == (k_scale, v_scale)
    for bad in (0.0, -1.0, float("inf"), float("nan"), 1e39):
        with pytest.raises(ValueError):
            fp8_e4m3_codec(k_scale=bad)


def test_half_ulp_and_metrics_on_hand_computed_values() -> None:
    assert half_ulp(np.array([1.0]), "bf16")[0] == 2**-8
    assert half_ulp(np.array([3.0]), "bf16")[0] == 2**-7
    assert half_ulp(np.array([1.0]), "fp16")[0] == 2**-11
    expected = np.array([1.0, 2.0, -4.0])
    report = parity_report(expected + np.array([0.0, 2**-7, 0.0]), expected, "bf16")
    assert report["max_abs"] == 2**-7
    assert report["max_abs_excess"] == 0.0  # 2^-7 is exactly half an ulp at 2
    assert report["rel_l2"] == pytest.approx(2**-7 / np.sqrt(21))


# --- plan and store: known answers from the reference's tests ------------------------------


@pytest.mark.parametrize("case", KNOWN["plan"], ids=lambda c: c["mode"])
def test_plan_known_answers(case: dict) -> None:
    result = paged.plan(case["mode"], case["rows"], case["lengths"], np.array(case["table"]), case["block_size"])
    assert result["request_of_row"].tolist() == case["request_of_row"]
    assert result["positions"].tolist() == case["positions"]
    assert result["slot_mapping"].tolist() == case["slot_mapping"]


@pytest.mark.parametrize("case", KNOWN["plan_refusals"], ids=lambda c: c["message"])
def test_plan_refusals(case: dict) -> None:
    with pytest.raises(paged.PlanError):
        paged.plan(case["mode"], case["rows"], case["lengths"], np.array(case["table"]), 4)


def test_plan_matches_a_token_walk() -> None:
    rng = np.random.default_rng(3)
    for _ in range(50):
        batch, bs = int(rng.integers(1, 6)), int(rng.choice([1, 4, 16]))
        lengths = [int(x) for x in rng.integers(0, 40, size=batch)]
        rows = [int(rng.integers(1, n + 1)) if n else int(rng.integers(0, 3)) for n in lengths]
        width = max(-(-n // bs) for n in lengths) or 1
        table = rng.integers(1, 99, size=(batch, width))
        result = paged.plan("mixed", rows, lengths, table, bs)
        slots = []
        for b, (count, n) in enumerate(zip(rows, lengths)):
            for j in range(count):
                if n == 0:
                    slots.append(0)
                    continue
                pos = n - count + j
                # walk the table a token at a time
                walked = 0
                for entry in table[b]:
                    if walked + bs > pos:
                        slots.append(int(entry) * bs + pos - walked)
                        break
                    walked += bs
        assert result["slot_mapping"].tolist() == slots


@pytest.mark.parametrize("layout", ["nhd", "hnd"])
@pytest.mark.parametrize("case", KNOWN["store"], ids=["two-requests", "padding"])
def test_store_known_answers(layout: str, case: dict) -> None:
    bs, hkv, d = case["block_size"], case["kv_heads"], case["head_dim"]
    shape = (case["blocks"], bs, hkv, d) if layout == "nhd" else (case["blocks"], hkv, bs, d)
    k_cache = np.full(shape, -1.0, dtype=np.float32)
    v_cache = np.full(shape, -1.0, dtype=np.float32)
    step = paged.plan("mixed", case["rows"], case["lengths"], np.array(case["table"]), bs)
    n = len(step["slot_mapping"])
    rng = np.random.default_rng(1)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    paged.store(k_cache, v_cache, k, v, step["slot_mapping"], layout)
    nk, nv = paged.nhd(k_cache, layout), paged.nhd(v_cache, layout)
    real = [i for i, (blk, off) in enumerate(case["landing"]) if (blk, off) != (0, 0)]
    for i in real:
        blk, off = case["landing"][i]
        assert np.array_equal(nk[blk, off], k[i]) and np.array_equal(nv[blk, off], v[i])
    written = {tuple(case["landing"][i]) for i in real}
    for blk in range(1, case["blocks"]):
        for off in range(bs):
            if (blk, off) not in written:
                assert (nk[blk, off] == -1.0).all() and (nv[blk, off] == -1.0).all()


def test_block_ops() -> None:
    rng = np.random.default_rng(2)
    k = rng.standard_normal((8, 4, 2, 8)).astype(np.float32)
    v = rng.standard_normal((8, 4, 2, 8)).astype(np.float32)
    gk, gv = paged.gather(k, v, np.array([5, 1, 5]))
    assert np.array_equal(gk, k[[5, 1, 5]]) and np.array_equal(gv, v[[5, 1, 5]])
    k2, v2 = k.copy(), v.copy()
    paged.copy_blocks(k2, v2, np.array([1, 2]), np.array([6, 7]))
    assert np.array_equal(k2[[6, 7]], k[[1, 2]]) and np.array_equal(k2[:6], k[:6])
    paged.zero_blocks(k2, v2, np.array([2, 4]))
    assert (k2[[2, 4]] == 0).all() and (v2[[2, 4]] == 0).all() and np.array_equal(k2[[0, 1, 3, 5]], k[[0, 1, 3, 5]])


# --- attention -----------------------------------------------------------------------------


TINY = [
    ("decode-one-block", [(1, 4), (1, 4)], "decode"),
    ("decode-ends-inside-blocks", [(1, 1), (1, 3), (1, 5), (1, 7), (1, 9)], "decode"),
    ("decode-with-padding", [(1, 6), (1, 0), (1, 2)], "decode"),
    ("prefill-chunks-and-verify", [(4, 4), (3, 11), (1 + 3, 9), (2, 0)], "mixed"),
]


@pytest.mark.parametrize("name,steps,mode", TINY, ids=[t[0] for t in TINY])
@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (4, 2), (6, 1), (8, 4)])
@pytest.mark.parametrize("layout", ["nhd", "hnd"])
def test_attention_matches_a_brute_force(name: str, steps: list, mode: str, heads: int, kv_heads: int, layout: str) -> None:
    s = build_scenario(steps, heads=heads, kv_heads=kv_heads, head_dim=8, layout=layout, mode=mode, seed=11)
    expected = brute_force(s)
    np.testing.assert_allclose(s.expected(np.float64), expected, rtol=0, atol=1e-12)
    np.testing.assert_allclose(s.expected(np.float32), expected, rtol=0, atol=2e-6)


@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (4, 2), (6, 1), (8, 4)])
def test_torch_decode_restatement_matches_the_brute_force(heads: int, kv_heads: int) -> None:
    # the CPU baseline's torch restatement of _attend_decode: whole padded tables (NaN in the
    # unused slots and block 0), a padding request, lengths ending inside blocks
    from oracle.torch_decode import attend_decode

    s = build_scenario([(1, 6), (1, 0), (1, 2), (1, 9), (1, 4)], heads=heads, kv_heads=kv_heads, head_dim=8,
                       mode="decode", seed=12)
    expected = brute_force(s)
    got = attend_decode(torch.from_numpy(s.q).double(), torch.from_numpy(paged.nhd(s.k, s.layout)).double(),
                        torch.from_numpy(paged.nhd(s.v, s.layout)).double(), torch.from_numpy(s.table),
                        torch.tensor(s.lengths), scale=s.scale)
    assert torch.isfinite(got).all()
    np.testing.assert_allclose(got.numpy(), expected, rtol=0, atol=2e-6)
    assert not got[1].any()


@pytest.mark.parametrize("layout", ["nhd", "hnd"])
def test_attention_of_requests_matches_attention(layout: str) -> None:
    # the shared-gather form used for full-size prefill chunks: the same outputs as attention()
    # (itself pinned by the brute force) on mixed steps with padding requests, rows ending
    # inside blocks, passes of rows that split a request, and NaN in every unused slot
    steps = [(5, 23), (1, 0), (9, 9), (3, 40), (1, 1), (2, 0), (17, 64)]
    for heads, kv_heads in ((8, 2), (6, 1), (4, 4)):
        s = build_scenario(steps, heads=heads, kv_heads=kv_heads, head_dim=16, block_size=8, layout=layout,
                           mode="mixed", seed=13)
        expected = s.expected(np.float64)
        for rows_per_pass in (1, 4, 64):
            got = paged.attention_of_requests(s.q, s.k, s.v, s.table, np.asarray(s.lengths), scale=s.scale,
                                              request_of_row=s.plan["request_of_row"],
                                              positions=s.plan["positions"], layout=layout,
                                              rows_per_pass=rows_per_pass)
            assert np.isfinite(got).all()
            np.testing.assert_allclose(got, expected, rtol=0, atol=1e-12)
    tiny = build_scenario([(4, 4), (2, 0), (3, 11)], heads=4, kv_heads=2, head_dim=8, mode="mixed", seed=11)
    got = paged.attention_of_requests(tiny.q, tiny.k, tiny.v, tiny.table, np.asarray(tiny.lengths),
                                      scale=tiny.scale, request_of_row=tiny.plan["request_of_row"],
                                      positions=tiny.plan["positions"])
    np.testing.assert_allclose(got, brute_force(tiny), rtol=0, atol=1e-12)


def test_attention_matches_torch_sdpa() -> None:
    steps = [(1, 70), (1, 17), (3, 40), (1, 1)]
    s = build_scenario(steps, heads=12, kv_heads=4, head_dim=64, block_size=16, seed=5)
    got = s.expected(np.float64)
    q, k, v = s.q, paged.nhd(s.k, s.layout), paged.nhd(s.v, s.layout)
    row = 0
    for b, (count, length) in enumerate(steps):
        pos = np.arange(length)
        blocks = s.table[b, pos // s.block_size]
        ck = torch.from_numpy(k[blocks, pos % s.block_size]).double().transpose(0, 1)  # [Hkv, L, D]
        cv = torch.from_numpy(v[blocks, pos % s.block_size]).double().transpose(0, 1)
        query = torch.from_numpy(q[row:row + count]).double().transpose(0, 1)  # [H, rows, D]
        mask = torch.arange(length)[None, :] <= torch.arange(length - count, length)[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(
            query, ck, cv, attn_mask=mask, scale=s.scale, enable_gqa=True
        )
        np.testing.assert_allclose(got[row:row + count], ref.transpose(0, 1).numpy(), rtol=0, atol=1e-12)
        row += count


def test_one_visible_key_returns_its_value_exactly() -> None:
    s = build_scenario([(1, 1)], heads=2, kv_heads=2, head_dim=8, mode="decode", dtype="fp16")
    got = s.expected(np.float32)
    blk = s.table[0, 0]
    assert np.array_equal(got[0], paged.nhd(s.v, s.layout)[blk, 0])


def test_scale_zero_gives_the_mean_of_the_visible_values() -> None:
    s = build_scenario([(2, 6)], heads=4, kv_heads=2, head_dim=8, scale=0.0)
    got = s.expected(np.float64)
    v = paged.nhd(s.v, s.layout)
    for row, visible in enumerate([5, 6]):
        pos = np.arange(visible)
        mean = v[s.table[0, pos // 4], pos % 4].astype(np.float64).mean(axis=0)
        np.testing.assert_allclose(got[row], np.repeat(mean, 2, axis=0), rtol=0, atol=1e-12)


def test_padding_rows_are_zero_and_nan_does_not_leak() -> None:
    s = build_scenario([(2, 6), (1, 0), (3, 0), (1, 5)], heads=4, kv_heads=2, head_dim=8)
    got = s.expected(np.float32)
    assert np.isfinite(got).all()
    assert not got[[2, 3, 4, 5]].any()


def test_the_physical_placement_of_blocks_does_not_matter() -> None:
    a = build_scenario([(1, 37), (1, 20)], head_dim=64, block_size=8, seed=9, mode="decode")
    # renumber the pool: a permutation of the blocks and of the table gives the same result
    perm = np.concatenate([[0], np.random.default_rng(4).permutation(np.arange(1, a.k_bits.shape[0]))])
    inverse = np.argsort(perm)
    moved_k, moved_v = a.k[inverse], a.v[inverse]
    table = perm[a.table] * (a.table > 0)
    got = paged.attention(a.q, moved_k, moved_v, table, np.array(a.lengths), scale=a.scale, precision=np.float64)
    np.testing.assert_array_equal(got, a.expected(np.float64))


def test_golden_fixture_is_reproduced() -> None:
    data = np.load(GOLDEN / "smollm2_small.npz")
    got = paged.attention(
        bits_to_f32(data["q"], "fp16"),
        bits_to_f32(data["k_cache"], "fp16"),
        bits_to_f32(data["v_cache"], "fp16"),
        data["table"],
        data["lengths"],
        scale=float(data["scale"]),
        precision=np.float64,
    )
    np.testing.assert_allclose(got, data["expected"], rtol=0, atol=1e-12)
