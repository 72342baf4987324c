"""Fused RoPE + KV append: HIP kernel vs the CPU oracle, bit for bit.

Ports test_triton_rope.py:8-50 of the reference (there: assert_close at the
bf16 default tolerance). Here every output — rotated q and k and the whole
cache, placement included — must equal the oracle's bits: the oracle is the
reference's torch path (apply_rope + store_kvcache) in bf16 on the CPU, whose
per-op rounding tests/test_oracle.py pins.
"""

import pytest
import torch

from oracle import rope as orope
from tests._cases import BLOCK_SIZE, tuned

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]


def _kernel():
    from babyvllm.kernels.rope import fused_rope_and_cache
    return fused_rope_and_cache


def _oracle(q, k, v, cos, sin, cache, slots):
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    qr, kr = orope.apply_rope(qc, kc, cos.cpu(), sin.cpu())
    cc = None
    if cache is not None:
        cc = cache.cpu().clone()
        orope.store_kvcache(kr, vc, cc, slots.cpu())
    return qr, kr, cc


def _bits_equal(a, b):
    return torch.equal(a.cpu().view(torch.int16), b.cpu().view(torch.int16))


def _qkv(T, H, Hkv, D, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    qkv = torch.randn(T, (H + 2 * Hkv) * D, device="cuda", dtype=torch.bfloat16, generator=g)
    q = qkv[:, : H * D].view(T, H, D)
    k = qkv[:, H * D: (H + Hkv) * D].view(T, Hkv, D)
    v = qkv[:, (H + Hkv) * D:].view(T, Hkv, D)
    return qkv, q, k, v


@pytest.mark.parametrize("T,H,Hkv,D", [(17, 28, 4, 128), (8, 14, 2, 64), (1, 28, 4, 128), (5, 4, 4, 256)])
def test_rope_and_cache_bitwise(T, H, Hkv, D):
    g = torch.Generator(device="cuda").manual_seed(42)
    q = torch.randn(T, H, D, device="cuda", dtype=torch.bfloat16, generator=g)
    k = torch.randn(T, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=g)
    v = torch.randn(T, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=g)
    cos = torch.randn(T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    sin = torch.randn(T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    nb = 10
    slots = torch.randperm(nb * BLOCK_SIZE, device="cuda", generator=g)[:T].to(torch.int64)
    cache = torch.randn(2, nb, BLOCK_SIZE, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=g)
    qr, kr, cr = _oracle(q, k, v, cos, sin, cache, slots)
    q2, k2 = _kernel()(q, k, v, cos, sin, cache, slots)
    torch.cuda.synchronize()
    assert q2.data_ptr() == q.data_ptr() and k2.data_ptr() == k.data_ptr()
    assert _bits_equal(q, qr) and _bits_equal(k, kr) and _bits_equal(cache, cr)


def test_views_into_fused_qkv_with_real_tables():
    """Model layout: q/k/v are strided views of one QKV row; cos/sin from RotaryEmbedding (θ = 1e6)."""
    from babyvllm.layers.rotary import RotaryEmbedding

    T, H, Hkv, D = 64, 28, 4, 128
    qkv, q, k, v = _qkv(T, H, Hkv, D, seed=1)
    assert not q.is_contiguous()
    rope = RotaryEmbedding(D, 4097, base=1e6).cuda()
    g = torch.Generator(device="cuda").manual_seed(2)
    pos = torch.randint(128, 4097, (T,), device="cuda", generator=g)
    cos, sin = rope(pos, torch.bfloat16)
    ct, st = orope.rope_tables(D, 4097, 1e6)
    assert torch.equal(cos.cpu(), ct[pos.cpu()].bfloat16()) and torch.equal(sin.cpu(), st[pos.cpu()].bfloat16())
    nb = 8192
    cache = torch.zeros(2, nb, BLOCK_SIZE, Hkv, D, device="cuda", dtype=torch.bfloat16)
    slots = torch.randperm(nb * BLOCK_SIZE, device="cuda", generator=g)[:T].to(torch.int64)
    before = qkv.clone()
    qr, kr, _ = _oracle(q, k, v, cos, sin, None, None)
    _kernel()(q, k, v, cos, sin, cache, slots)
    torch.cuda.synchronize()
    assert _bits_equal(q, qr) and _bits_equal(k, kr)
    assert _bits_equal(v, before[:, (H + Hkv) * D:].view(T, Hkv, D))  # v is read, never written
    flat = cache.view(2, -1, Hkv, D)
    assert _bits_equal(flat[0, slots], kr) and _bits_equal(flat[1, slots], v)
    assert int((flat.abs().sum(dim=(2, 3)) != 0).sum()) <= 2 * T  # nothing else written


def test_prefill_8192_tokens_placement_and_rotation():
    """Config 2b: 64 sequences × 128 new tokens at positions 0..127, slots from seeded tables."""
    from babyvllm.layers.rotary import RotaryEmbedding

    S, N, H, Hkv, D, nb = 64, 128, 28, 4, 128, 8192
    T = S * N
    qkv, q, k, v = _qkv(T, H, Hkv, D, seed=3)
    g = torch.Generator().manual_seed(4)
    tables = torch.randperm(nb, generator=g)[: S * (N // BLOCK_SIZE)].view(S, N // BLOCK_SIZE)
    pos = torch.arange(N).repeat(S)
    seq = torch.arange(S).repeat_interleave(N)
    slots = (tables[seq, pos // BLOCK_SIZE] * BLOCK_SIZE + pos % BLOCK_SIZE).to(torch.int64)
    rope = RotaryEmbedding(D, 4096, base=1e6).cuda()
    cos, sin = rope(pos.cuda(), torch.bfloat16)
    cache = torch.zeros(2, nb, BLOCK_SIZE, Hkv, D, device="cuda", dtype=torch.bfloat16)
    qr, kr, _ = _oracle(q, k, v, cos, sin, None, None)
    vr = v.cpu().clone()
    _kernel()(q, k, v, cos, sin, cache, slots.cuda())
    torch.cuda.synchronize()
    assert _bits_equal(q, qr) and _bits_equal(k, kr)
    # Read every sequence back through its table (slot = table[pos//16]·16 + pos%16).
    kc = cache[0].cpu()[tables].reshape(S, N, Hkv, D)
    vc = cache[1].cpu()[tables].reshape(S, N, Hkv, D)
    assert _bits_equal(kc.reshape(T, Hkv, D), kr) and _bits_equal(vc.reshape(T, Hkv, D), vr)


def test_no_cache_rotates_only():
    T, H, Hkv, D = 9, 28, 4, 128
    qkv, q, k, v = _qkv(T, H, Hkv, D, seed=5)
    g = torch.Generator(device="cuda").manual_seed(6)
    cos = torch.randn(T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    sin = torch.randn(T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    vbefore = v.clone()
    qr, kr, _ = _oracle(q, k, v, cos, sin, None, None)
    _kernel()(q, k, v, cos, sin)
    torch.cuda.synchronize()
    assert _bits_equal(q, qr) and _bits_equal(k, kr) and _bits_equal(v, vbefore)


def test_unaligned_views_take_the_scalar_path_with_the_same_bits():
    T, H, Hkv, D = 6, 28, 4, 128
    g = torch.Generator(device="cuda").manual_seed(7)
    buf = torch.randn(T * (H + 2 * Hkv) * D + 1, device="cuda", dtype=torch.bfloat16, generator=g)
    qkv = buf[1:].view(T, (H + 2 * Hkv) * D)  # 2-byte misaligned base
    q = qkv[:, : H * D].view(T, H, D)
    k = qkv[:, H * D: (H + Hkv) * D].view(T, Hkv, D)
    v = qkv[:, (H + Hkv) * D:].view(T, Hkv, D)
    cos = torch.randn(T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    sin = torch.randn(T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    cache = torch.zeros(2, 4, BLOCK_SIZE, Hkv, D, device="cuda", dtype=torch.bfloat16)
    slots = torch.tensor([3, 17, 40, 0, 63, 22], device="cuda", dtype=torch.int64)
    qr, kr, cr = _oracle(q, k, v, cos, sin, cache, slots)
    _kernel()(q, k, v, cos, sin, cache, slots)
    torch.cuda.synchronize()
    assert _bits_equal(q, qr) and _bits_equal(k, kr) and _bits_equal(cache, cr)


def test_out_of_range_slots_are_not_written():
    T, H, Hkv, D = 4, 28, 4, 128
    qkv, q, k, v = _qkv(T, H, Hkv, D, seed=8)
    g = torch.Generator(device="cuda").manual_seed(9)
    cos = torch.randn(T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    sin = torch.randn(T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    cache = torch.zeros(2, 2, BLOCK_SIZE, Hkv, D, device="cuda", dtype=torch.bfloat16)
    slots = torch.tensor([5, -1, 32, 31], device="cuda", dtype=torch.int64)  # 32 = num_slots
    qr, kr, _ = _oracle(q, k, v, cos, sin, None, None)
    _kernel()(q, k, v, cos, sin, cache, slots)
    torch.cuda.synchronize()
    assert _bits_equal(q, qr) and _bits_equal(k, kr)
    flat = cache.view(2, -1, Hkv, D).cpu()
    assert _bits_equal(flat[0, 5], kr[0]) and _bits_equal(flat[0, 31], kr[3])
    others = [s for s in range(32) if s not in (5, 31)]
    assert flat[:, others].abs().sum() == 0


def test_rejects_wrong_dtypes_and_cpu_tensors():
    T, H, Hkv, D = 2, 4, 2, 64
    q = torch.randn(T, H, D, device="cuda", dtype=torch.float32)
    k = torch.randn(T, Hkv, D, device="cuda", dtype=torch.bfloat16)
    cos = torch.randn(T, D, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        _kernel()(q, k, k, cos, cos)
    with pytest.raises(RuntimeError):
        _kernel()(q.cpu().bfloat16(), k.cpu(), k.cpu(), cos.cpu(), cos.cpu())


@pytest.mark.parametrize("seed", range(12))
def test_random_steps_bitwise(seed):
    """Seeded random steps: 1-600 tokens, random head shapes, q/k/v as views of
    one fused QKV row or as separate tensors, scattered slots, with or without
    the cache; every output bit-equal to the oracle."""
    g = torch.Generator().manual_seed(4000 + seed)
    H, Hkv, D = [(28, 4, 128), (14, 2, 64), (8, 8, 128), (12, 2, 64), (32, 8, 128)][seed % 5]
    T = int(torch.randint(1, 601, (1,), generator=g))
    fused = bool(torch.randint(2, (1,), generator=g))
    with_cache = seed % 4 != 3
    gd = torch.Generator(device="cuda").manual_seed(seed)
    if fused:
        _, q, k, v = _qkv(T, H, Hkv, D, seed)
    else:
        q = torch.randn(T, H, D, device="cuda", dtype=torch.bfloat16, generator=gd)
        k = torch.randn(T, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=gd)
        v = torch.randn(T, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=gd)
    pos = torch.randint(0, 8192, (T,), generator=g).to("cuda")
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32, device="cuda") / D))
    ang = pos[:, None].float() * inv[None]
    cos = torch.cat([ang.cos(), ang.cos()], -1).to(torch.bfloat16)
    sin = torch.cat([ang.sin(), ang.sin()], -1).to(torch.bfloat16)
    cache = slots = None
    if with_cache:
        nb = (T + BLOCK_SIZE - 1) // BLOCK_SIZE + 3
        cache = torch.randn(2, nb, BLOCK_SIZE, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=gd)
        slots = torch.randperm(nb * BLOCK_SIZE, generator=g)[:T].to(torch.int64).to("cuda")
    qr, kr, cr = _oracle(q, k, v, cos, sin, cache, slots)
    _kernel()(q, k, v, cos, sin, cache, slots)
    torch.cuda.synchronize()
    assert _bits_equal(q, qr) and _bits_equal(k, kr)
    if with_cache:
        assert _bits_equal(cache, cr)


# The two aligned append kernels (bvllm_set_tuning knob 5): 0 = head rows per
# wave (the default), 1 = one thread per 16-byte chunk pair. Same bits.
_LAYOUTS = [0, 1]


def _special_values(n, g):
    """bf16 values that stress rounding: ±inf, NaN of both signs, the largest
    finite values, subnormals, signed zeros and ordinary normals."""
    special = torch.tensor([float("inf"), float("-inf"), float("nan"), -float("nan"),
                            3.3895e38, -3.3895e38, 1e-39, -1e-39, 9.2e-41, 0.0, -0.0, 1.0],
                           dtype=torch.float32).bfloat16()
    x = torch.randn(n, generator=g).bfloat16()
    pick = torch.randint(0, 3, (n,), generator=g) == 0
    x[pick] = special[torch.randint(0, special.numel(), (int(pick.sum()),), generator=g)]
    return x


@pytest.mark.parametrize("layout", _LAYOUTS)
def test_special_values_bitwise(layout):
    """inf, NaN, overflow and subnormal inputs (q, k, cos, sin): NaN exactly where
    the oracle has NaN, every other output bit equal to the oracle's. (A NaN's
    sign and payload are not compared: torch's own CPU kernels store 0x7fc0 on
    their scalar path and 0xffff on their vector path.)"""
    T, H, Hkv, D = 24, 28, 4, 128
    g = torch.Generator().manual_seed(11)
    q = _special_values(T * H * D, g).view(T, H, D).cuda()
    k = _special_values(T * Hkv * D, g).view(T, Hkv, D).cuda()
    v = _special_values(T * Hkv * D, g).view(T, Hkv, D).cuda()
    cos = _special_values(T * D, g).view(T, D).cuda()
    sin = _special_values(T * D, g).view(T, D).cuda()
    cache = torch.zeros(2, 4, BLOCK_SIZE, Hkv, D, device="cuda", dtype=torch.bfloat16)
    slots = torch.randperm(4 * BLOCK_SIZE, generator=g)[:T].to(torch.int64).cuda()
    qr, kr, cr = _oracle(q, k, v, cos, sin, cache, slots)
    with tuned(5, layout):
        _kernel()(q, k, v, cos, sin, cache, slots)
        torch.cuda.synchronize()
    for got, want in ((q, qr), (k, kr), (cache[0], cr[0])):
        got, want = got.cpu(), want.cpu()
        nan = want.isnan()
        assert torch.equal(got.isnan(), nan)
        assert torch.equal(got[~nan].view(torch.int16), want[~nan].view(torch.int16))
    # V rows are copied, not computed: every bit, NaN sign and payload included,
    # and untouched slots stay zero.
    assert torch.equal(cache[1].cpu().view(torch.int16), cr[1].view(torch.int16))
    assert torch.equal(cache[1].view(-1, Hkv, D)[slots].cpu().view(torch.int16), v.cpu().view(torch.int16))


@pytest.mark.parametrize("layout", _LAYOUTS)
@pytest.mark.parametrize("H,Hkv,D,T", [(28, 4, 128, 37), (14, 2, 64, 9), (8, 8, 128, 5), (4, 4, 256, 3),
                                       (32, 8, 128, 2), (12, 2, 64, 1)])
def test_layouts_give_the_same_bits(layout, H, Hkv, D, T):
    _, q, k, v = _qkv(T, H, Hkv, D, seed=T)
    g = torch.Generator(device="cuda").manual_seed(T + 1)
    cos = torch.randn(T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    sin = torch.randn(T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    nb = (T + BLOCK_SIZE - 1) // BLOCK_SIZE + 2
    cache = torch.randn(2, nb, BLOCK_SIZE, Hkv, D, device="cuda", dtype=torch.bfloat16, generator=g)
    slots = torch.randperm(nb * BLOCK_SIZE, device="cuda", generator=g)[:T].to(torch.int64)
    slots[0] = -1  # out-of-range slot: not written
    qr, kr, _ = _oracle(q, k, v, cos, sin, None, None)
    cr = cache.cpu().clone()
    orope.store_kvcache(kr[1:], v.cpu()[1:], cr, slots.cpu()[1:])
    with tuned(5, layout):
        _kernel()(q, k, v, cos, sin, cache, slots)
        torch.cuda.synchronize()
    assert _bits_equal(q, qr) and _bits_equal(k, kr) and _bits_equal(cache, cr)
