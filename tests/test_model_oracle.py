"""Pinning the oracle's non-attention ops (oracle/model_oracle.c) and the CPU Qwen3 forward -- CPU only.

Each op is checked against something other than its own formula:
  * linear / RMSNorm: the reference's own golden files (testdata/linear_case.bin, norm_case.bin, copied to
    tests/golden/ref_*.bin) at the reference test's tolerance (src/module/linear.zig, src/module/norm.zig:
    |got - ref| <= 1e-3 + 1e-3 |ref|); a case where f32 summation order changes the result (pins "index order");
    the rounding point of Qwen3RMSNorm written with torch ((x * rsqrt).to(bf16) * w);
  * RoPE: the complex-number rotation in float64, position 0 = identity, relative-position invariance of q.k,
    the table against float64 numpy (theta ** (-2i/d), a different formula);
  * SiLU / add / mul: float64 closed forms and torch's bf16 arithmetic;
  * sampling: numpy argmax (first index of the maximum), explicit ties, NaN, all -inf, SplitMix64's published
    first output for state 0 (0xE220A8397B1DCDAF), Gumbel-max frequencies against softmax;
  * the CPU forward: a decode step after a prefill gives bit-identical logits to a prefill of the whole
    sequence (KV cache, positions and block tables wired consistently).
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def bf16(x) -> np.ndarray:
    t = torch.tensor(np.asarray(x, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def f32(b) -> np.ndarray:
    return O.bf16_to_f32(b)


def _read_case(name, dims):
    raw = open(os.path.join(GOLDEN, name), "rb").read()
    hdr = np.frombuffer(raw[:12], "<i4")
    return hdr, np.frombuffer(raw[12:], "<f4")


# ---------------------------------------------------------------- linear
def test_linear_reference_golden_case():
    (S, K, N), body = _read_case("ref_linear_case.bin", 3)
    x = body[:S * K].reshape(S, K)
    w = body[S * K:S * K + N * K].reshape(N, K)
    y_ref = body[S * K + N * K:].reshape(S, N)
    y = O.linear(x, w)
    assert y.dtype == np.float32
    assert np.all(np.abs(y - y_ref) <= 1e-3 + 1e-3 * np.abs(y_ref))


def test_linear_sums_in_index_order():
    # (2^24 + 1) + 1 rounds to 2^24 twice in f32; any other order (or pairwise sums) gives 2^24 + 2
    x = np.array([[1.0, 1.0, 1.0]], np.float32)
    w = np.array([[2.0 ** 24, 1.0, 1.0]], np.float32)
    assert O.linear(x, w)[0, 0] == 2.0 ** 24
    assert O.linear(x[:, ::-1].copy(), w[:, ::-1].copy())[0, 0] == 2.0 ** 24 + 2


def test_linear_bf16_small_integers_exact():
    rng = np.random.default_rng(0)
    x = rng.integers(-4, 5, (9, 40)).astype(np.float32)
    w = rng.integers(-4, 5, (13, 40)).astype(np.float32)
    y = O.linear(bf16(x), bf16(w))
    assert y.dtype == np.uint16
    np.testing.assert_array_equal(f32(y), (x @ w.T).astype(np.float32))  # |y| <= 640: exact in bf16


# ---------------------------------------------------------------- RMSNorm
def test_rmsnorm_reference_golden_case():
    hdr, body = _read_case("ref_norm_case.bin", 3)
    S, H = int(hdr[0]), int(hdr[1])
    eps = float(np.frombuffer(np.int32(hdr[2]).tobytes(), "<f4")[0])
    assert abs(eps - 1e-6) < 1e-12
    x = body[:S * H].reshape(S, H)
    g = body[S * H:S * H + H]
    y_ref = body[S * H + H:].reshape(S, H)
    y = O.rmsnorm(x, g, eps)
    assert np.all(np.abs(y - y_ref) <= 1e-3 + 1e-3 * np.abs(y_ref))


def test_rmsnorm_bf16_rounding_point_matches_qwen3_norm():
    rng = np.random.default_rng(1)
    x = bf16(rng.standard_normal((64, 1024)) * 3)
    g = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    g_b = f32(bf16(g))  # torch multiplies bf16 * bf16 weight; use a bf16-representable gain
    y = O.rmsnorm(x, g_b, 1e-6)
    xt = torch.tensor(f32(x))
    normed = (xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    yt = (normed * torch.tensor(g_b).to(torch.bfloat16)).view(torch.int16).numpy().view(np.uint16)
    diff = np.abs(f32(y) - f32(yt))
    # rsqrt vs 1/sqrt and the mean's summation order differ by an ulp of f32 at most: a few bf16 flips
    assert (y == yt).mean() > 0.99
    assert np.all(diff <= np.abs(f32(yt)) * 2 ** -7)


# ---------------------------------------------------------------- RoPE
def test_rope_table_against_float64():
    c, s = O.rope_table(300, 128, 1e6)
    i = np.arange(64)
    ang = np.arange(300)[:, None] * (1e6 ** (-2.0 * i / 128))[None, :]
    np.testing.assert_allclose(c[:, :64], np.cos(ang), rtol=0, atol=6e-8)
    np.testing.assert_allclose(s[:, :64], np.sin(ang), rtol=0, atol=6e-8)
    assert np.array_equal(c[:, :64], c[:, 64:]) and np.array_equal(s[:, :64], s[:, 64:])
    assert np.all(c[0] == 1) and np.all(s[0] == 0)


def test_rope_is_neox_complex_rotation():
    rng = np.random.default_rng(2)
    T, nh, hd = 7, 3, 128
    x = rng.standard_normal((T, nh, hd)).astype(np.float32)
    pos = np.array([0, 1, 5, 17, 100, 255, 3], np.int32)
    c, s = O.rope_table(256, hd, 1e6)
    y = O.rope(x, pos, c, s)
    half = hd // 2
    z = (x[..., :half] + 1j * x[..., half:]).astype(np.complex128)
    ang = pos[:, None, None] * (1e6 ** (-2.0 * np.arange(half) / hd))[None, None, :]
    zr = z * np.exp(1j * ang)
    np.testing.assert_allclose(y[..., :half], zr.real, atol=2e-6)
    np.testing.assert_allclose(y[..., half:], zr.imag, atol=2e-6)
    np.testing.assert_array_equal(y[0], x[0])  # position 0: cos 1, sin 0 -> exact identity


def test_rope_relative_position_invariance():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 1, 128)).astype(np.float32)
    k = rng.standard_normal((1, 1, 128)).astype(np.float32)
    c, s = O.rope_table(512, 128, 1e4)
    dots = []
    for m, n in ((10, 3), (110, 103), (400, 393)):
        qr = O.rope(q, np.array([m], np.int32), c, s)
        kr = O.rope(k, np.array([n], np.int32), c, s)
        dots.append(float((qr * kr).sum()))
    assert max(dots) - min(dots) < 1e-3


def test_rope_bf16_in_place_alias_and_tail_dims():
    rng = np.random.default_rng(4)
    x = bf16(rng.standard_normal((3, 2, 16)))
    c, s = O.rope_table(8, 8, 1e4)
    y = O.rope(x, np.array([1, 2, 3], np.int32), c, s, rope_dim=8)
    np.testing.assert_array_equal(y[..., 8:], x[..., 8:])  # dims past rope_dim are copied


# ---------------------------------------------------------------- elementwise
def test_silu_against_float64():
    v = np.linspace(-30, 30, 20001, dtype=np.float32)
    y = O.silu(v)
    ref = v.astype(np.float64) / (1 + np.exp(-v.astype(np.float64)))
    np.testing.assert_allclose(y, ref, rtol=3e-7, atol=1e-30)
    yb = O.silu(bf16(v))
    tb = torch.nn.functional.silu(torch.tensor(f32(bf16(v)))).to(torch.bfloat16)
    assert (yb == tb.view(torch.int16).numpy().view(np.uint16)).mean() > 0.999


def test_add_mul_match_torch_bf16_and_broadcast():
    rng = np.random.default_rng(5)
    a = bf16(rng.standard_normal((6, 64)) * 10)
    b = bf16(rng.standard_normal((6, 64)))
    ta, tb = torch.tensor(f32(a)).to(torch.bfloat16), torch.tensor(f32(b)).to(torch.bfloat16)
    u16 = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    np.testing.assert_array_equal(O.add(a, b), u16(ta + tb))
    np.testing.assert_array_equal(O.mul(a, b), u16(ta * tb))
    row = b[0]
    np.testing.assert_array_equal(O.add(a, row), u16(ta + tb[0]))


def test_embedding_and_gather():
    rng = np.random.default_rng(6)
    table = bf16(rng.standard_normal((50, 16)))
    ids = np.array([3, 0, 49, 3], np.int32)
    np.testing.assert_array_equal(O.embedding(ids, table), table[ids])
    with pytest.raises(IndexError):
        O.embedding(np.array([50], np.int32), table)
    x = bf16(rng.standard_normal((9, 16)))
    np.testing.assert_array_equal(O.gather(x, [8, 0, 4]), x[[8, 0, 4]])


# ---------------------------------------------------------------- sampling
def test_splitmix64_published_value():
    assert O.splitmix64(0) == 0xE220A8397B1DCDAF


def test_greedy_sample_ties_nan_and_empty():
    rng = np.random.default_rng(7)
    lg = rng.standard_normal((5, 1000)).astype(np.float32)
    lg[1, [10, 500, 999]] = 9.0  # tie: the first index wins
    lg[2, :] = -np.inf
    lg[3, 7] = np.nan
    lg[3, 8] = 50.0
    lg[4, :] = np.nan
    ids = O.sample(lg)
    assert ids[0] == np.argmax(lg[0]) and ids[1] == 10 and ids[2] == 0 and ids[3] == 8 and ids[4] == 0
    b = bf16(lg[:2])
    assert list(O.sample(b)) == [int(np.argmax(f32(b[0]))), 10]


def test_gumbel_sample_follows_softmax():
    logits = np.log(np.array([[0.5, 0.3, 0.15, 0.05]], np.float32))
    counts = np.zeros(4)
    for seed in range(4000):
        counts[O.sample(logits, np.array([1.0], np.float32), seed=seed)[0]] += 1
    np.testing.assert_allclose(counts / counts.sum(), [0.5, 0.3, 0.15, 0.05], atol=0.03)
    # temperature 0 is greedy whatever the seed
    assert O.sample(logits, np.array([0.0], np.float32), seed=123)[0] == 0


# ---------------------------------------------------------------- CPU Qwen3 forward
def _tiny():
    from llmgen_amd.qwen3 import Qwen3Config, random_weights

    cfg = Qwen3Config(vocab=512, hidden=128, n_layers=2, n_head=4, n_kv_head=2, head_dim=32, ffn=256,
                      max_model_len=128, block_size=16)
    return cfg, random_weights(cfg, seed=3, std=0.1, embd_row_sigma=1.0)


def test_cpu_forward_decode_equals_prefill_of_whole_sequence():
    from llmgen_amd import step as S
    from oracle.qwen3_ref import Qwen3Ref

    cfg, W = _tiny()
    mb = cfg.max_model_len // cfg.block_size
    rng = np.random.default_rng(8)
    toks = rng.integers(0, cfg.vocab, 21).tolist()
    table = [5, 2, 7, 0, 1, 3, 4, 6]
    # prefill 20 tokens, then decode token 21
    a = Qwen3Ref(cfg, W, num_blocks=8)
    a.forward(S.fill_meta([S.Entry(0, 20, table)], cfg.block_size, mb, 64), toks[:20], mb)
    ids_a, lg_a = a.forward(S.fill_meta([S.Entry(20, 1, table)], cfg.block_size, mb, 64), toks[20:], mb,
                            return_logits=True)
    # one prefill of all 21 tokens, other block table
    b = Qwen3Ref(cfg, W, num_blocks=8)
    ids_b, lg_b = b.forward(S.fill_meta([S.Entry(0, 21, [1, 0, 3, 2, 5, 4, 7, 6])], cfg.block_size, mb, 64), toks,
                            mb, return_logits=True)
    np.testing.assert_array_equal(lg_a, lg_b)
    assert list(ids_a) == list(ids_b)
    # the host-side tables equal the oracle's
    from llmgen_amd.qwen3 import rope_tables

    c1, s1 = rope_tables(cfg.max_model_len, cfg.head_dim, cfg.rope_theta)
    c2, s2 = O.rope_table(cfg.max_model_len, cfg.head_dim, cfg.rope_theta)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2)
