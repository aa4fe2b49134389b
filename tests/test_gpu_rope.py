"""RoPE forward/backward parity of the HIP kernel (through the C ABI) with the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from gpu_util import BF16, close, close_fp32, from_npz, randn
from oracle import rope as o_rope
from picotron_amd import ops

pytestmark = pytest.mark.gpu

LAYOUTS = ["interleaved", "rotate_half"]


def _bhsd_view(b, s, h, d, dtype, device, seed):
    """(B, H, S, D) view of (B, S, H, D) memory, as attention's _split_heads produces."""

    return randn((b, s, h, d), dtype, device, seed).transpose(1, 2)


def test_golden_fixture(gpu):
    f = np.load(GOLDEN / "rope_small.npz")
    x, cos, sin = (from_npz(f[k], gpu) for k in ("x", "cos", "sin"))
    for layout in LAYOUTS:
        y, _ = ops.rope(x, cos, sin, layout=layout)
        inv, _ = ops.rope(x, cos, sin, layout=layout, inverse=True)
        close_fp32(y, from_npz(f[f"y_{layout}"], gpu))
        close_fp32(inv, from_npz(f[f"inv_{layout}"], gpu))


def test_fp32_matches_reference_fallback(gpu):
    # interleaved fp32 on a (B, H, S, D) contiguous tensor vs the reference eager path
    x = randn((2, 4, 64, 32), torch.float32, gpu, 1)
    dy = randn((2, 4, 64, 32), torch.float32, gpu, 2)
    cos, sin = o_rope.tables(64, 32, 10_000.0, device=gpu)
    y, _ = ops.rope(x, cos, sin)
    dx, _ = ops.rope(dy, cos, sin, inverse=True)
    fy, fdx = o_rope.fallback_forward_backward(x.cpu(), cos.cpu(), sin.cpu(), dy.cpu())
    close_fp32(y, fy)
    close_fp32(dx, fdx)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_full_config_bf16(gpu, layout):
    # q [8, 2048, 32, 128], k [8, 2048, 8, 128] bf16 in (B, S, H, D) memory, theta 5e5
    q = _bhsd_view(8, 2048, 32, 128, torch.bfloat16, gpu, 11)
    k = _bhsd_view(8, 2048, 8, 128, torch.bfloat16, gpu, 12)
    cos, sin = o_rope.tables(2048, 128, 500_000.0, device=gpu)
    yq, yk = ops.rope(q, cos, sin, layout=layout, x1=k)
    assert yq.stride() == q.stride() and yk.stride() == k.stride()  # memory layout kept
    close(yq, o_rope.rotate(q, cos, sin, layout, compute=torch.float32), torch.bfloat16)
    close(yk, o_rope.rotate(k, cos, sin, layout, compute=torch.float32), torch.bfloat16)
    dq = _bhsd_view(8, 2048, 32, 128, torch.bfloat16, gpu, 13)
    dk = _bhsd_view(8, 2048, 8, 128, torch.bfloat16, gpu, 14)
    gq, gk = ops.rope(dq, cos, sin, layout=layout, inverse=True, x1=dk)
    close(gq, o_rope.rotate(dq, cos, sin, layout, inverse=True, compute=torch.float32), torch.bfloat16)
    close(gk, o_rope.rotate(dk, cos, sin, layout, inverse=True, compute=torch.float32), torch.bfloat16)
    # size-independent: per-(row, pair) norms are preserved to bf16 rounding
    torch.testing.assert_close(yq.float().norm(dim=-1), q.float().norm(dim=-1), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [2, 6, 16, 64, 96, 128, 256])
def test_head_dims(gpu, layout, dtype, head_dim):
    x = randn((2, 3, 17, head_dim), dtype, gpu, head_dim)
    cos, sin = o_rope.tables(20, head_dim, 10_000.0, device=gpu)  # table longer than seq
    y, _ = ops.rope(x, cos, sin, layout=layout)
    close(y, o_rope.rotate(x, cos, sin, layout), dtype)
    back, _ = ops.rope(y, cos, sin, layout=layout, inverse=True)
    close(back, o_rope.rotate(o_rope.rotate(x, cos, sin, layout).to(dtype), cos, sin, layout, inverse=True), dtype)


def test_strided_unaligned_and_gqa(gpu):
    cos, sin = o_rope.tables(33, 64, 500_000.0, device=gpu)
    base = randn((2, 33, 6, 64 + 1), torch.bfloat16, gpu, 3)
    x = base[..., 1:].transpose(1, 2)  # odd strides and a 2-byte offset: element path
    y, _ = ops.rope(x, cos, sin, layout="rotate_half")
    close(y, o_rope.rotate(x, cos, sin, "rotate_half"), torch.bfloat16)
    q = _bhsd_view(2, 33, 8, 64, torch.bfloat16, gpu, 4)
    k = _bhsd_view(2, 33, 2, 64, torch.bfloat16, gpu, 5)
    yq, yk = ops.rope(q, cos, sin, x1=k)
    close(yq, o_rope.rotate(q, cos, sin), torch.bfloat16)
    close(yk, o_rope.rotate(k, cos, sin), torch.bfloat16)
    empty = torch.empty((2, 0, 33, 64), dtype=torch.bfloat16, device=gpu)
    ye, _ = ops.rope(empty, cos, sin)
    assert ye.shape == empty.shape


@pytest.mark.parametrize("layout", LAYOUTS)
def test_fused_qkv_projection_views(gpu, layout):
    # q and k as views of one fused QKV projection output (B, S, (Hq + 2 Hkv) * D): their
    # sequence stride spans every head of q, k and v, and k starts Hq * D elements in
    from picotron_amd.nn.triton_kernels import triton_apply_rotary_embedding_pair

    b, s, hq, hkv, d = 2, 40, 8, 2, 128
    width = (hq + 2 * hkv) * d
    qkv = randn((b, s, width), torch.bfloat16, gpu, 21).requires_grad_(True)
    q = qkv[..., : hq * d].view(b, s, hq, d).transpose(1, 2)
    k = qkv[..., hq * d : (hq + hkv) * d].view(b, s, hkv, d).transpose(1, 2)
    cos, sin = o_rope.tables(s, d, 500_000.0, device=gpu)
    rq, rk = triton_apply_rotary_embedding_pair(q, k, cos, sin, layout=layout)
    torch.testing.assert_close(rq.double(), o_rope.rotate(q.detach(), cos, sin, layout), **BF16)
    torch.testing.assert_close(rk.double(), o_rope.rotate(k.detach(), cos, sin, layout), **BF16)
    gq = randn(rq.shape, torch.bfloat16, gpu, 22)
    gk = randn(rk.shape, torch.bfloat16, gpu, 23)
    torch.autograd.backward((rq, rk), (gq, gk))
    want = torch.zeros((b, s, width), dtype=torch.float64, device=gpu)
    want[..., : hq * d] = o_rope.rotate(gq, cos, sin, layout, inverse=True).transpose(1, 2).reshape(b, s, hq * d)
    want[..., hq * d : (hq + hkv) * d] = (
        o_rope.rotate(gk, cos, sin, layout, inverse=True).transpose(1, 2).reshape(b, s, hkv * d))
    torch.testing.assert_close(qkv.grad.double(), want, **BF16)  # v's columns get no gradient


@pytest.mark.parametrize("layout", LAYOUTS)
def test_autograd_surface_and_module(gpu, layout):
    import warnings

    from picotron_amd.nn import RotaryEmbedding

    q = _bhsd_view(2, 48, 8, 64, torch.bfloat16, gpu, 6).requires_grad_(True)
    k = _bhsd_view(2, 48, 4, 64, torch.bfloat16, gpu, 7).requires_grad_(True)
    rope = RotaryEmbedding(64, 500_000.0, use_triton_rope=True, layout=layout)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        rq, rk = rope(q, k)
    assert not rope._triton_fallback_warned
    cos, sin = o_rope.tables(48, 64, 500_000.0, device=gpu)
    torch.testing.assert_close(rq.double(), o_rope.rotate(q.detach(), cos, sin, layout), **BF16)
    gq = randn(rq.shape, torch.bfloat16, gpu, 8)
    gk = randn(rk.shape, torch.bfloat16, gpu, 9)
    torch.autograd.backward((rq, rk), (gq, gk))
    torch.testing.assert_close(q.grad.double(), o_rope.rotate(gq, cos, sin, layout, inverse=True), **BF16)
    torch.testing.assert_close(k.grad.double(), o_rope.rotate(gk, cos, sin, layout, inverse=True), **BF16)


def test_module_shares_one_table_across_sequence_lengths(gpu):
    from picotron_amd.nn import RotaryEmbedding

    rope = RotaryEmbedding(64, 500_000.0, use_triton_rope=True, layout="rotate_half")
    for seq in (48, 17, 96, 40):  # shorter lengths read a prefix of the longest table so far
        q = _bhsd_view(2, seq, 4, 64, torch.bfloat16, gpu, seq)
        k = _bhsd_view(2, seq, 2, 64, torch.bfloat16, gpu, seq + 1)
        rq, rk = rope(q, k)
        cos, sin = o_rope.tables(seq, 64, 500_000.0, device=gpu)
        torch.testing.assert_close(rq.double(), o_rope.rotate(q, cos, sin, "rotate_half"), **BF16)
        torch.testing.assert_close(rk.double(), o_rope.rotate(k, cos, sin, "rotate_half"), **BF16)
    assert not rope._triton_fallback_warned
    assert len(rope._fp32_tables) == 1
    assert next(iter(rope._fp32_tables.values()))[0].size(0) == 96
