"""GPU parity of the dense kernels (linear, prefill attention) against the oracle.

Bars: fp32 within 1e-5 relative.  bf16 linear: every output within one bf16
ulp of the exact (fp64) product of the same bf16 inputs, and within one ulp of
the oracle's own bf16 result (both round an fp32 accumulation once, so they
may differ by that rounding).  bf16 attention: 2e-2 absolute.
"""

from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_bf16_close, assert_fp32_close, generator
from oracle import kernels as ref

pytestmark = pytest.mark.gpu


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    # Spacing of bf16 numbers at |x| (8 significant bits).
    mag = x.abs().clamp_min(2.0**-126)
    return torch.exp2(torch.floor(torch.log2(mag)) - 7)


def _check_linear_bf16(actual, x, w, b, *, against_oracle=True):
    exact = x.double() @ w.double().T
    if b is not None:
        exact = exact + b.double()
    oracle = ref.linear(x, w, b).double()
    a = actual.double().cpu()
    # One bf16 ulp for the final rounding plus the worst-case error of an fp32
    # accumulation of K products, K * 2^-24 * sum|x w| (Higham's bound): near
    # a rounding tie the fp32 sum may land on either side.
    accumulation = x.shape[-1] * 2.0**-24 * (x.double().abs() @ w.double().abs().T)
    tol = _bf16_ulp(exact) * 1.0 + accumulation + 1e-6
    assert ((a - exact).abs() <= tol).all(), float((a - exact).abs().max())
    if against_oracle:
        tol_o = _bf16_ulp(oracle) * 1.0 + 1e-6
        assert ((a - oracle).abs() <= tol_o + _bf16_ulp(exact)).all()
    return float((a == oracle).double().mean())


@pytest.mark.parametrize("rows", [1, 8, 33, 64, 128, 1000])
@pytest.mark.parametrize(
    "k,n,bias",
    [(896, 896, True), (896, 128, True), (896, 4864, False), (4864, 896, False),
     (2048, 6000, True)],
)
def test_linear_bf16_qwen_shapes(gpu, rows, k, n, bias):
    from stateful_llm_compiler_hip.backends import hip_linear

    announce(f"linear bf16 M={rows} K={k} N={n} bias={bias}")
    g = generator(rows * 13 + k + n)
    x = torch.randn(rows, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16()
    b = (torch.randn(n, generator=g) * 0.02).bfloat16() if bias else None
    y = hip_linear(x.to(gpu), w.to(gpu), None if b is None else b.to(gpu))
    torch.cuda.synchronize()
    _check_linear_bf16(y, x, w, b)


@pytest.mark.parametrize("rows,k,n,strided", [(8, 896, 151936, False), (1, 896, 20000, False),
                                              (16, 2048, 17000, False), (8, 896, 20000, True),
                                              (24, 896, 20000, False)])
def test_linear_bf16_vocabulary_width(gpu, rows, k, n, strided):
    """The vocabulary-width decode kernel (one wave per 16 features over all
    of K; input rows staged in LDS when they are 16-byte aligned, read from
    the cache otherwise, as a strided view here; rows past 16 take two
    row blocks) within one bf16 ulp of the fp64 product."""
    from stateful_llm_compiler_hip.backends import hip_linear

    announce(f"linear bf16 vocabulary width M={rows} K={k} N={n} strided={strided}")
    g = generator(rows + k + n)
    x = torch.randn(rows, k + (3 if strided else 0), generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16()
    xd, wd = x.to(gpu), w.to(gpu)
    if strided:
        # Row stride k + 3 and a 2-byte offset, through the C ABI (the
        # Python wrapper takes contiguous inputs only).
        from stateful_llm_compiler_hip import _native

        x, xd = x[:, 1:k + 1], xd[:, 1:k + 1]
        y = torch.empty(rows, n, dtype=torch.bfloat16, device=gpu)
        status = _native.library().slc_hip_linear(
            xd.data_ptr(), wd.data_ptr(), None, y.data_ptr(), _native.SLC_BF16, rows, n, k,
            k + 3, n, _native.current_stream(xd.device))
        _native.check(status, "slc_hip_linear")
    else:
        y = hip_linear(xd, wd)
    torch.cuda.synchronize()
    _check_linear_bf16(y, x, w, None, against_oracle=False)


def test_linear_bf16_large_m_and_3d(gpu):
    from stateful_llm_compiler_hip.backends import hip_linear

    announce("linear bf16 3-D input [4, 1024, 896] -> 896")
    g = generator(3)
    x = torch.randn(4, 1024, 896, generator=g).bfloat16()
    w = (torch.randn(896, 896, generator=g) * 0.02).bfloat16()
    b = (torch.randn(896, generator=g) * 0.02).bfloat16()
    y = hip_linear(x.to(gpu), w.to(gpu), b.to(gpu))
    torch.cuda.synchronize()
    assert y.shape == (4, 1024, 896)
    _check_linear_bf16(y.reshape(-1, 896), x.reshape(-1, 896), w, b)


@pytest.mark.parametrize("k,n", [(896, 4864), (4864, 896)])
def test_linear_bf16_bench_rows(gpu, k, n):
    # Config 4's largest GEMM rows (M = 8 x 4096), the shape the bench times;
    # checked in row blocks against the fp64 product and the oracle.
    from stateful_llm_compiler_hip.backends import hip_linear

    announce(f"linear bf16 M=32768 K={k} N={n}")
    g = generator(k + 2 * n)
    x = torch.randn(32768, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16()
    # The bar is the exact (fp64) product: every output within one bf16 ulp.
    # The CPU oracle's bf16 GEMM itself strays past one ulp of it at K = 4864,
    # so its agreement is reported, not bounded.
    y = hip_linear(x.to(gpu), w.to(gpu)).cpu()
    agree = [_check_linear_bf16(y[start:start + 4096], x[start:start + 4096], w, None,
                                against_oracle=False) for start in range(0, 32768, 4096)]
    print(f"bitwise agreement with the oracle: {sum(agree) / len(agree):.4f}")


TILES = ("t128x128", "t128x64", "t64x128", "t64x64", "t32x64", "r128x128", "r256x128", "r128x64", "r64x64",
         "s256x128")


@pytest.mark.parametrize("rows,k,n,bias", [(4096, 896, 128, True), (300, 896, 896, True),
                                           (1000, 4864, 896, False), (77, 200, 136, True),
                                           (520, 896, 4864, False), (1100, 896, 9728, True)])
def test_linear_tiles_are_bit_identical_and_exact(gpu, rows, k, n, bias):
    """Every GEMM tile variant a plan may pick: within the fp64 product's bar
    and bit-identical to every other tile (same k order per output)."""

    from stateful_llm_compiler_hip.backends import hip_linear

    g = generator(rows + 7 * k + n)
    x = torch.randn(rows, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16()
    b = (torch.randn(n, generator=g) * 0.02).bfloat16() if bias else None
    xg, wg, bg = x.to(gpu), w.to(gpu), None if b is None else b.to(gpu)
    outputs = {}
    for tile in TILES:
        announce(f"linear tile {tile} M={rows} K={k} N={n}")
        outputs[tile] = hip_linear(xg, wg, bg, tile=tile)
        torch.cuda.synchronize()
    _check_linear_bf16(outputs["t128x128"], x, w, b)
    for tile in TILES[1:]:
        assert torch.equal(outputs[tile], outputs["t128x128"]), tile


@pytest.mark.parametrize("rows,n", [(1000, 151936), (4096, 4864)])
def test_linear_persistent_tile_equals_ring_tile(gpu, rows, n):
    """The persistent 256 x 128 kernel over grids many rounds deep (a
    vocabulary-wide head, ragged M) gives the ring kernel's bits."""

    from stateful_llm_compiler_hip.backends import hip_linear

    announce(f"linear persistent tile M={rows} N={n}")
    g = torch.Generator(device=gpu).manual_seed(rows + n)
    x = torch.randn(rows, 896, device=gpu, generator=g, dtype=torch.bfloat16)
    w = torch.randn(n, 896, device=gpu, generator=g, dtype=torch.bfloat16) * 0.02
    got = hip_linear(x, w, tile="s256x128")
    want = hip_linear(x, w, tile="r256x128")
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.isfinite(got.float()).all()
    xh, wh = x.half(), w.half()
    bh = torch.randn(n, device=gpu, generator=g, dtype=torch.float16) * 0.02
    got = hip_linear(xh, wh, bh, tile="s256x128")
    want = hip_linear(xh, wh, bh, tile="r256x128")
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_linear_persistent_tile_with_unaligned_output(gpu):
    """The persistent tile stores 8 bytes per lane from registers: an output
    whose base is 2 bytes off 16-byte alignment takes the staged-store
    kernel instead, with the same bits."""

    from stateful_llm_compiler_hip import _native
    from stateful_llm_compiler_hip.backends import hip_linear

    rows, n, k = 1100, 9728, 896
    announce(f"linear persistent tile, unaligned output M={rows} N={n}")
    g = torch.Generator(device=gpu).manual_seed(5)
    x = torch.randn(rows, k, device=gpu, generator=g, dtype=torch.bfloat16)
    w = torch.randn(n, k, device=gpu, generator=g, dtype=torch.bfloat16) * 0.02
    want = hip_linear(x, w, tile="r256x128")
    flat = torch.full((rows * n + 1,), float("nan"), device=gpu, dtype=torch.bfloat16)
    got = flat[1:].view(rows, n)
    status = _native.library().slc_hip_linear_tile(
        x.data_ptr(), w.data_ptr(), None, got.data_ptr(), _native.SLC_BF16, rows, n, k, k, n,
        _native.LINEAR_TILES["s256x128"], _native.current_stream(x.device))
    _native.check(status, "slc_hip_linear_tile")
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_linear_tile_plan_reaches_the_c_abi(gpu, monkeypatch):
    """A profile plan's tile choice is the tile argument slc_hip_linear_tile
    receives (recorded by a pass-through proxy of the loaded library)."""

    from stateful_llm_compiler_hip import _native
    from stateful_llm_compiler_hip.cost_model import KernelProfile
    from stateful_llm_compiler_hip.execution import HipExecutor

    lib = _native.library()
    calls = []

    class Proxy:
        def __getattr__(self, name):
            return getattr(lib, name)

        def slc_hip_linear_tile(self, *args):
            calls.append(args[10])
            return lib.slc_hip_linear_tile(*args)

    profile = KernelProfile.from_dict({"schema_version": 1, "linear": [
        {"rows": 512, "out_features": 128, "in_features": 896, "dtype": "bf16",
         "hip_variants": {"t128x128": 12.0, "t32x64": 9.0}},
        {"rows": 32768, "out_features": 128, "in_features": 896, "dtype": "bf16",
         "hip_variants": {"t128x128": 22.0, "t32x64": 28.0}}]})
    plan = profile.plan("linear", out_features=128, in_features=896, dtype="bf16")
    g = generator(11)
    w = (torch.randn(128, 896, generator=g) * 0.02).bfloat16().to(gpu)
    small = torch.randn(512, 896, generator=g).bfloat16().to(gpu)
    large = torch.randn(32768, 896, generator=g).bfloat16().to(gpu)
    executor = HipExecutor()
    announce("linear tile plan through the executor")
    monkeypatch.setattr(_native, "_library", Proxy())
    y_small = executor._linear([small, w], {"has_bias": False, "tile_plan": plan})
    y_large = executor._linear([large, w], {"has_bias": False, "tile_plan": plan})
    y_auto = executor._linear([small, w], {"has_bias": False})
    torch.cuda.synchronize()
    monkeypatch.undo()
    tiles = _native.LINEAR_TILES
    assert calls == [tiles["t32x64"], tiles["t128x128"], tiles["auto"]]
    assert torch.equal(y_small, y_auto)
    _check_linear_bf16(y_large[:4096], large[:4096].cpu(), w.cpu(), None, against_oracle=False)


@pytest.mark.parametrize("k", [72, 40, 100])
def test_linear_bf16_k_tails(gpu, k):
    from stateful_llm_compiler_hip.backends import hip_linear

    announce(f"linear bf16 K tail K={k}")
    g = generator(k)
    x = torch.randn(70, k, generator=g).bfloat16()
    w = (torch.randn(130, k, generator=g) * 0.1).bfloat16()
    y = hip_linear(x.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    _check_linear_bf16(y, x, w, None)


def test_linear_fp16(gpu):
    from stateful_llm_compiler_hip.backends import hip_linear

    announce("linear fp16")
    g = generator(7)
    x = torch.randn(40, 512, generator=g).half()
    w = (torch.randn(1536, 512, generator=g) * 0.05).half()
    b = (torch.randn(1536, generator=g) * 0.05).half()
    y = hip_linear(x.to(gpu), w.to(gpu), b.to(gpu)).cpu().double()
    exact = x.double() @ w.double().T + b.double()
    # fp16 ulp: 11 significant bits
    ulp = torch.exp2(torch.floor(torch.log2(exact.abs().clamp_min(2.0**-14))) - 10)
    assert ((y - exact).abs() <= ulp + 1e-6).all()


@pytest.mark.parametrize("rows", [1, 3, 17])
def test_linear_fp32(gpu, rows):
    from stateful_llm_compiler_hip.backends import hip_linear

    announce(f"linear fp32 M={rows}")
    g = generator(rows)
    x = torch.randn(rows, 896, generator=g)
    w = torch.randn(4864, 896, generator=g) * 0.02
    b = torch.randn(4864, generator=g) * 0.02
    y = hip_linear(x.to(gpu), w.to(gpu), b.to(gpu))
    torch.cuda.synchronize()
    assert_fp32_close(y, ref.linear(x, w, b))


# -------------------------------------------------------- prefill attention


def _prefill_case(gpu, batch, tokens, dtype, seed, *, mask_kind, causal, q_heads=14, kv_heads=2, head_dim=64,
                  mask_dtype=torch.float32, scale=None, softmax_order="online"):
    from stateful_llm_compiler_hip.backends import hip_prefill_attention

    g = generator(seed)
    # Projection-layout views ([B, T, H, D] transposed), as the model produces them.
    q = torch.randn(batch, tokens, q_heads, head_dim, generator=g).to(dtype).transpose(1, 2)
    k = torch.randn(batch, tokens, kv_heads, head_dim, generator=g).to(dtype).transpose(1, 2)
    v = torch.randn(batch, tokens, kv_heads, head_dim, generator=g).to(dtype).transpose(1, 2)
    if mask_kind == "none":
        mask = None
    elif mask_kind == "causal":
        future = torch.triu(torch.ones(tokens, tokens, dtype=torch.bool), diagonal=1)
        mask = torch.zeros(batch, 1, tokens, tokens).masked_fill(future, float("-inf"))
    elif mask_kind == "zeros":
        mask = torch.zeros(batch, 1, tokens, tokens)
    else:
        mask = torch.randn(batch, 1, tokens, tokens, generator=g)
    if mask is not None:
        mask = mask.to(mask_dtype)
    scale = head_dim**-0.5 if scale is None else scale
    expected = ref.prefill_attention(
        q, k, v, mask, groups=q_heads // kv_heads, scale=scale, causal=causal
    )

    def dev(t):
        return t.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)

    actual = hip_prefill_attention(
        dev(q), dev(k), dev(v), None if mask is None else mask.to(gpu),
        scale=scale, causal=causal, softmax_order=softmax_order,
    )
    torch.cuda.synchronize()
    return actual.cpu(), expected


@pytest.mark.parametrize("batch,tokens", [(1, 7), (2, 64), (1, 100), (2, 128), (1, 1024)])
def test_prefill_causal_flag_bf16(gpu, batch, tokens):
    announce(f"prefill bf16 causal=True no mask B={batch} T={tokens}")
    actual, expected = _prefill_case(gpu, batch, tokens, torch.bfloat16, tokens, mask_kind="none", causal=True)
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("batch,kind", [(2, "causal"), (8, "none")])
def test_prefill_bench_shapes_bf16(gpu, batch, kind):
    """Config 4's longest prompts (T = 4096) at the shapes the bench times:
    the causal flag at B = 8 and an explicit causal [B, 1, T, T] mask at
    B = 2.  The oracle runs one (batch row, kv head) at a time so its fp32
    score matrix stays at 7 x 4096 x 4096."""

    from stateful_llm_compiler_hip.backends import hip_prefill_attention

    tokens, q_heads, kv_heads, head_dim = 4096, 14, 2, 64
    groups = q_heads // kv_heads
    announce(f"prefill bf16 B={batch} T={tokens} mask={kind}")
    g = generator(batch + tokens)
    q = torch.randn(batch, q_heads, tokens, head_dim, generator=g).bfloat16()
    k = torch.randn(batch, kv_heads, tokens, head_dim, generator=g).bfloat16()
    v = torch.randn(batch, kv_heads, tokens, head_dim, generator=g).bfloat16()
    mask = None
    if kind == "causal":
        future = torch.triu(torch.ones(tokens, tokens, dtype=torch.bool), diagonal=1)
        mask = torch.zeros(batch, 1, tokens, tokens).masked_fill(future, float("-inf"))
    causal = kind == "none"
    actual = hip_prefill_attention(q.to(gpu), k.to(gpu), v.to(gpu),
                                   None if mask is None else mask.to(gpu),
                                   scale=head_dim ** -0.5, causal=causal).cpu()
    for b in range(batch):
        for h in range(kv_heads):
            heads = slice(h * groups, (h + 1) * groups)
            expected = ref.prefill_attention(
                q[b:b + 1, heads], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1],
                None if mask is None else mask[b:b + 1], groups=groups,
                scale=head_dim ** -0.5, causal=causal)
            assert_bf16_close(actual[b:b + 1, heads], expected)


@pytest.mark.parametrize("tokens", [7, 130])
def test_prefill_mask_provides_causality_bf16(gpu, tokens):
    # causal="mask": the reference passes the causal -inf mask (qwen2.py:540-573).
    announce(f"prefill bf16 causal mask T={tokens}")
    actual, expected = _prefill_case(gpu, 2, tokens, torch.bfloat16, 5, mask_kind="causal", causal=False)
    assert_bf16_close(actual, expected)


def test_prefill_mask_and_flag_bf16(gpu):
    announce("prefill bf16 random mask + causal flag")
    actual, expected = _prefill_case(gpu, 2, 96, torch.bfloat16, 6, mask_kind="random", causal=True)
    assert_bf16_close(actual, expected)


def test_prefill_bidirectional_zero_mask_bf16(gpu):
    # Reference case: an all-zero mask is bidirectional attention
    # (test_prefill_attention.py:97-114).
    announce("prefill bf16 zero mask bidirectional")
    actual, expected = _prefill_case(gpu, 2, 80, torch.bfloat16, 7, mask_kind="zeros", causal=False)
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("q_heads,kv_heads", [(14, 2), (8, 1), (4, 4), (8, 4), (16, 4)])
@pytest.mark.parametrize("tokens", [7, 64, 100, 257])
@pytest.mark.parametrize(
    "variant", ["causal-flag", "bf16-causal-mask", "f32-random-mask-causal", "f16-zeros", "bidirectional"]
)
def test_prefill_grouped_kernel(gpu, q_heads, kv_heads, tokens, variant):
    # GQA groups of 7, 8, 1, 2 and 4 heads take the grouped-head kernel, with
    # no mask, a 2-byte mask, or an fp32 mask (all with unit key stride).
    # "bidirectional" (no mask, no causal flag) bounds the last tile by the
    # token count alone.
    announce(f"prefill grouped QH{q_heads} KVH{kv_heads} T={tokens} {variant}")
    kind, causal, mdt = {
        "causal-flag": ("none", True, torch.float32),
        "bidirectional": ("none", False, torch.float32),
        "bf16-causal-mask": ("causal", False, torch.bfloat16),
        "f32-random-mask-causal": ("random", True, torch.float32),
        "f16-zeros": ("zeros", False, torch.float16),
    }[variant]
    dtype = torch.float16 if variant == "f16-zeros" else torch.bfloat16
    actual, expected = _prefill_case(gpu, 2, tokens, dtype, tokens + q_heads, mask_kind=kind, causal=causal,
                                     q_heads=q_heads, kv_heads=kv_heads, mask_dtype=mdt)
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("scale", [0.1, 0.3, 0.25])
def test_prefill_grouped_kernel_scale(gpu, scale):
    # A scale that is not a power of two rounds the scaled score a second
    # time (as the reference executor does); 0.25 takes the single-rounding
    # path.
    announce(f"prefill grouped scale={scale}")
    actual, expected = _prefill_case(gpu, 2, 130, torch.bfloat16, 11, mask_kind="random", causal=True,
                                     scale=scale)
    assert_bf16_close(actual, expected)


def _equal_fraction(actual, expected):
    return float((actual.float() == expected.float()).float().mean())


@pytest.mark.parametrize("q_heads,kv_heads,tokens,kind,causal,dtype", [
    (14, 2, 7, "none", True, torch.bfloat16),        # config-1 prompt shape
    (14, 2, 300, "causal", False, torch.bfloat16),   # explicit causal mask
    (14, 2, 257, "random", True, torch.bfloat16),    # mask + flag, ragged tiles
    (8, 4, 130, "zeros", False, torch.float16),      # bidirectional, groups of 2
    (6, 2, 65, "none", True, torch.bfloat16),        # groups of 3: generic kernel
])
def test_prefill_exact_softmax_order(gpu, q_heads, kv_heads, tokens, kind, causal, dtype):
    """The exact order (normalise, round, then P.V) reproduces the reference
    executor's rounding: nearly every element equals the oracle bit for bit
    (what differs is the last bit of a q.k sum or an exp), and more of them
    than with the online order."""

    announce(f"prefill exact order QH{q_heads} KVH{kv_heads} T={tokens} {kind} causal={causal} {dtype}")
    args = dict(mask_kind=kind, causal=causal, q_heads=q_heads, kv_heads=kv_heads,
                mask_dtype=torch.float32)
    exact, expected = _prefill_case(gpu, 2, tokens, dtype, tokens + 5, softmax_order="exact", **args)
    online, _ = _prefill_case(gpu, 2, tokens, dtype, tokens + 5, softmax_order="online", **args)
    assert_bf16_close(exact, expected)
    e, o = _equal_fraction(exact, expected), _equal_fraction(online, expected)
    print(f"bitwise-equal fraction: exact {e:.4f}, online {o:.4f}")
    assert e >= 0.97 and e > o


def test_prefill_exact_order_fully_masked_row_is_nan(gpu):
    # A query row whose keys are all -inf: NaN, as the reference's softmax.
    from stateful_llm_compiler_hip.backends import hip_prefill_attention

    announce("prefill exact order fully masked row")
    g = generator(5)
    q = torch.randn(1, 14, 70, 64, generator=g).bfloat16().to(gpu)
    k = torch.randn(1, 2, 70, 64, generator=g).bfloat16().to(gpu)
    v = torch.randn(1, 2, 70, 64, generator=g).bfloat16().to(gpu)
    mask = torch.zeros(1, 1, 70, 70)
    mask[0, 0, 3] = float("-inf")
    out = hip_prefill_attention(q, k, v, mask.to(gpu), scale=0.125, softmax_order="exact")
    torch.cuda.synchronize()
    out = out.cpu().float()
    assert torch.isnan(out[0, :, 3]).all()
    assert not torch.isnan(out[0, :, :3]).any() and not torch.isnan(out[0, :, 4:]).any()


def test_prefill_fp32_generic(gpu):
    announce("prefill fp32 causal mask T=33 QH4 KVH2 D64")
    actual, expected = _prefill_case(gpu, 2, 33, torch.float32, 8, mask_kind="causal", causal=False, q_heads=4)
    assert_fp32_close(actual, expected)


def test_prefill_fp16_head_dim_128_generic(gpu):
    announce("prefill fp16 D=128 (generic)")
    actual, expected = _prefill_case(gpu, 1, 40, torch.float16, 9, mask_kind="none", causal=True, q_heads=4, head_dim=128)
    assert_bf16_close(actual, expected)


@pytest.mark.parametrize("m,n,k", [(300, 200, 128), (129, 136, 64), (77, 8, 192)])
def test_linear_bf16_partial_tiles(gpu, m, n, k):
    # Row and column tiles cut by M and N (N a multiple of 8: the 16-byte
    # store epilogue), K a multiple of the 64-wide k-tile.
    from stateful_llm_compiler_hip.backends import hip_linear

    announce(f"linear bf16 partial tiles M={m} N={n} K={k}")
    g = generator(m + n + k)
    x = torch.randn(m, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.05).bfloat16()
    b = (torch.randn(n, generator=g) * 0.05).bfloat16()
    y = hip_linear(x.to(gpu), w.to(gpu), b.to(gpu))
    torch.cuda.synchronize()
    _check_linear_bf16(y, x, w, b)


# ------------------------------------------------ mask tile classes (prefill)


def _class_masks(batch, tokens, dtype, seed):
    """Masks whose tiles cover every class: the causal mask, a left-padded
    causal mask (padding keys -inf for some rows), a block-sparse mask
    (random -inf tiles among random values), and a causal mask written with
    -0 in place of +0 (not the causal pattern bit for bit: class 2)."""

    g = generator(seed)
    future = torch.triu(torch.ones(tokens, tokens, dtype=torch.bool), diagonal=1)
    causal = torch.zeros(batch, 1, tokens, tokens).masked_fill(future, float("-inf"))
    padded = causal.clone()
    for b in range(batch):
        padded[b, :, :, : 37 * b] = float("-inf")
    tiles = -(-tokens // 64)
    dead = torch.rand(batch, tiles, tiles, generator=g) < 0.4
    sparse = torch.randn(batch, 1, tokens, tokens, generator=g)
    sparse = sparse.masked_fill(dead.repeat_interleave(64, 1).repeat_interleave(64, 2)[:, None, :tokens, :tokens],
                                float("-inf"))
    negzero = torch.full((batch, 1, tokens, tokens), -0.0).masked_fill(future, float("-inf"))
    return {name: m.to(dtype) for name, m in
            (("causal", causal), ("padded", padded), ("sparse", sparse), ("negzero", negzero))}


def _classes_reference(mask: torch.Tensor) -> torch.Tensor:
    """The class definition, restated on the host over the bit patterns."""

    batch, _, tokens, _ = mask.shape
    tiles = -(-tokens // 64)
    width = {2: torch.int16, 4: torch.int32}[mask.element_size()]
    bits = mask[:, 0].contiguous().view(width).long()
    ninf = int(torch.tensor(float("-inf"), dtype=mask.dtype).view(width))
    q = torch.arange(tokens).view(-1, 1)
    k = torch.arange(tokens).view(1, -1)
    pattern = torch.where(k <= q, torch.zeros((), dtype=torch.long), torch.tensor(ninf))
    out = torch.empty(batch, tiles, tiles, dtype=torch.uint8)
    for b in range(batch):
        for i in range(tiles):
            for j in range(tiles):
                blk = bits[b, 64 * i:64 * (i + 1), 64 * j:64 * (j + 1)]
                pat = pattern[64 * i:64 * (i + 1), 64 * j:64 * (j + 1)]
                out[b, i, j] = 0 if bool((blk == ninf).all()) else (1 if torch.equal(blk, pat) else 2)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("tokens", [64, 100, 200, 512])  # 100 in bf16/fp16: the scalar-load path
def test_prefill_mask_tile_classes(gpu, dtype, tokens):
    from stateful_llm_compiler_hip.backends import hip_prefill_mask_tiles

    for name, mask in _class_masks(3, tokens, dtype, tokens).items():
        announce(f"prefill mask tile classes {name} {dtype} T={tokens}")
        classes = hip_prefill_mask_tiles(mask.to(gpu)).cpu()
        expected = _classes_reference(mask)
        assert torch.equal(classes, expected), name
        if name == "causal":
            # below the diagonal 1, above 0, the diagonal tile 1
            assert int(classes.max()) == 1 and bool((classes[:, 0, 1:] == 0).all() if classes.shape[1] > 1 else True)
        if name == "negzero":
            assert bool((classes <= 2).all()) and int(classes.max()) == 2


@pytest.mark.parametrize("tokens", [200, 512])
@pytest.mark.parametrize("order", ["online", "exact"])
@pytest.mark.parametrize("causal", [False, True])
def test_prefill_mask_classes_are_bit_identical(gpu, tokens, order, causal):
    """Skipping dead tiles and applying causal-pattern tiles from indices
    gives the same bits as loading and adding every mask tile (classes all
    2), and both are within the bf16 bar of the oracle."""

    from stateful_llm_compiler_hip.backends import hip_prefill_attention

    batch, q_heads, kv_heads, head_dim = 3, 14, 2, 64
    g = generator(tokens + 3)
    q = torch.randn(batch, q_heads, tokens, head_dim, generator=g).bfloat16()
    k = torch.randn(batch, kv_heads, tokens, head_dim, generator=g).bfloat16()
    v = torch.randn(batch, kv_heads, tokens, head_dim, generator=g).bfloat16()
    tiles = -(-tokens // 64)
    every = torch.full((batch, tiles, tiles), 2, dtype=torch.uint8, device=gpu)
    for mask_dtype in (torch.bfloat16, torch.float32):
        for name, mask in _class_masks(batch, tokens, mask_dtype, 9).items():
            announce(f"prefill classes bitwise {name} {mask_dtype} T={tokens} order={order} causal={causal}")
            args = (q.to(gpu), k.to(gpu), v.to(gpu), mask.to(gpu))
            fast = hip_prefill_attention(*args, scale=0.125, causal=causal, softmax_order=order)
            slow = hip_prefill_attention(*args, scale=0.125, causal=causal, softmax_order=order,
                                         mask_tiles=every)
            torch.cuda.synchronize()
            assert torch.equal(fast.view(torch.int16), slow.view(torch.int16)), name
            if mask_dtype == torch.float32 and name in ("padded", "sparse"):
                expected = ref.prefill_attention(q, k, v, mask, groups=q_heads // kv_heads, scale=0.125,
                                                  causal=causal)
                finite = torch.isfinite(expected)
                assert torch.equal(finite, torch.isfinite(fast.cpu().float()))
                assert_bf16_close(fast.cpu()[finite], expected[finite])


@pytest.mark.parametrize("kind", ["causal-online", "mask-exact", "mask-online", "none-exact"])
def test_prefill_short_and_long_workgroups_agree(gpu, kind):
    """Short grids take 16-query workgroups, deeper ones 32-query workgroups
    (at most two 32-query workgroups per CU picks the short form).  Batch
    rows are independent, so a batch of 9 (32-query form on a 256-CU part)
    and its first 8 rows (16-query form) give the same bits for those rows."""

    from stateful_llm_compiler_hip.backends import hip_prefill_attention, hip_prefill_mask_tiles

    batch, q_heads, kv_heads, tokens, head_dim = 9, 14, 2, 1024, 64
    announce(f"prefill short/long workgroups {kind} T={tokens}")
    g = torch.Generator(device=gpu).manual_seed(17)
    q = torch.randn(batch, q_heads, tokens, head_dim, device=gpu, generator=g, dtype=torch.bfloat16)
    k = torch.randn(batch, kv_heads, tokens, head_dim, device=gpu, generator=g, dtype=torch.bfloat16)
    v = torch.randn(batch, kv_heads, tokens, head_dim, device=gpu, generator=g, dtype=torch.bfloat16)
    structure, order = kind.split("-")
    causal = structure == "causal"
    mask = None
    if structure == "mask":
        future = torch.ones(tokens, tokens, dtype=torch.bool, device=gpu).triu(1)
        mask = torch.zeros(tokens, tokens, device=gpu, dtype=torch.bfloat16).masked_fill(future, float("-inf"))
        mask = mask.expand(batch, 1, tokens, tokens).contiguous()

    def run(rows):
        m = None if mask is None else mask[:rows].contiguous()
        tiles = None if m is None else hip_prefill_mask_tiles(m)
        return hip_prefill_attention(q[:rows].contiguous(), k[:rows].contiguous(), v[:rows].contiguous(), m,
                                     scale=0.125, causal=causal, softmax_order=order, mask_tiles=tiles)

    long_form = run(9)
    short_form = run(8)
    torch.cuda.synchronize()
    assert torch.isfinite(short_form.float()).all()
    assert torch.equal(long_form[:8].view(torch.int16), short_form.view(torch.int16))
