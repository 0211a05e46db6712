"""Packed low-bit storage on the GPU: crbq_pack / crbq_unpack byte-for-byte
against the NumPy statement of the format (tests/packed_ref.py), exception
lists included, and bit-exact round trips of layers quantized by the block
loop; crbq_gemv_packed / crbq_gemm_packed against float64 products of the
unpacked weights; PackedLinear and the stack driver's pack option.

GEMV bar: |y - y64| <= 1e-5 * sum_c |w_c x_c| per output (fp32 sums of
exact 16-bit products)."""
import numpy as np
import pytest
import torch

from packed_ref import pack_ref, structured, unpack_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _k():
    from crb_amd import kernels
    return kernels


def _q16(q, dtype):
    bits = q.view(np.uint16)
    if dtype == torch.bfloat16:          # reinterpret the same bit patterns as bf16
        return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(q).to(DEV)


@pytest.mark.parametrize("R,C,dtype,n_odd", [(37, 300, torch.float16, 0),
                                             (64, 512, torch.bfloat16, 0),
                                             (5, 128, torch.float16, 3),
                                             (200, 1000, torch.bfloat16, 40)])
def test_pack_matches_format_statement(R, C, dtype, n_odd):
    print(f"pack structured {R}x{C} {dtype} odd={n_odd}", flush=True)
    q, masks = structured(R, C, seed=R + C, dtype=np.float16, n_odd=n_odd)
    bits = q.view(np.uint16)
    Q = _q16(q, dtype)
    M = torch.from_numpy(masks).to(DEV)
    codes, lut, sal, ex = _k().pack(Q, M)
    rc, rl, rs, rex, st = pack_ref(bits, masks, bf16=dtype == torch.bfloat16)
    assert st == 0 and (len(rex[0]) > 0) == (n_odd > 0)
    assert np.array_equal(codes.cpu().numpy(), rc)
    assert np.array_equal(lut.cpu().view(torch.int16).numpy().view(np.uint16), rl)
    assert np.array_equal(sal.cpu().numpy(), rs)
    assert np.array_equal(ex.idx.cpu().numpy(), rex[0])
    assert np.array_equal(ex.val.cpu().view(torch.int16).numpy().view(np.uint16), rex[1])
    assert np.array_equal(ex.delta.cpu().numpy(), rex[2])
    back = _k().unpack(codes, lut, sal, C, ex)
    assert torch.equal(back.view(torch.int16).cpu(), Q.view(torch.int16).cpu())


def test_pack_reports_structure_errors():
    print("pack errors", flush=True)
    from crb_amd._lib import CrbqError
    q, masks = structured(8, 256, seed=3)
    col = int(np.nonzero(masks[2, :128] == 1)[0][0])
    bad = q.copy()
    bad[2, col] = np.float16(0.123)            # one out-of-table value: an exception
    codes, lut, sal, ex = _k().pack(torch.from_numpy(bad).to(DEV), torch.from_numpy(masks).to(DEV))
    assert ex.idx.tolist() == [2 * 256 + col]
    with pytest.raises(CrbqError, match="exception list"):
        _k().pack(torch.from_numpy(bad).to(DEV), torch.from_numpy(masks).to(DEV), ex_cap=0)
    m2 = masks.copy()
    m2[5, int(np.nonzero(masks[0, :128] == 3)[0][0])] = 1
    with pytest.raises(CrbqError, match="salient columns differ"):
        _k().pack(torch.from_numpy(q).to(DEV), torch.from_numpy(m2).to(DEV))
    # a valid layer afterwards still packs (the status word is cleared per call)
    _k().pack(torch.from_numpy(q).to(DEV), torch.from_numpy(masks).to(DEV))


@pytest.mark.parametrize("method,dtype,R,C", [("crb", torch.float16, 96, 320),
                                              ("braq", torch.bfloat16, 64, 384),
                                              ("crbog", torch.float16, 48, 256)])
def test_quantized_layer_round_trip(method, dtype, R, C):
    """Layers from the block loop (LayerQuantizer with keep_masks) pack and
    unpack bit for bit (C = 320: a ragged last block of 64 columns, above the
    salient search's 50-column minimum)."""
    print(f"pack quantized {method} {R}x{C}", flush=True)
    from crb_amd.driver import LayerQuantizer, Sublayer
    g = torch.Generator().manual_seed(R * C)
    W = (torch.randn(R, C, generator=g) * 0.02).to(dtype).to(DEV)
    X = (torch.randn(4, 256, C, generator=g) * torch.exp(torch.randn(C, generator=g))).to(dtype)
    lq = LayerQuantizer([Sublayer("w", W, "x")], method=method, keep_masks=True)
    lq.add_batch("x", X.to(DEV))
    lq.quantize()
    codes, lut, sal, ex = _k().pack(W, lq.masks["w"])
    assert torch.equal(_k().unpack(codes, lut, sal, C, ex).view(torch.int16), W.view(torch.int16))
    rc, rl, rs, rex, st = pack_ref(W.view(torch.int16).cpu().numpy().view(np.uint16),
                                   lq.masks["w"].cpu().numpy(), bf16=dtype == torch.bfloat16)
    assert st == 0 and np.array_equal(codes.cpu().numpy(), rc)
    assert np.array_equal(ex.idx.cpu().numpy(), rex[0])


@pytest.mark.parametrize("R,C,dtype,nvec", [(37, 300, torch.float16, 1),
                                            (256, 1024, torch.float16, 3),
                                            (130, 640, torch.bfloat16, 8),
                                            (1000, 4096, torch.bfloat16, 1),
                                            (512, 2000, torch.float16, 5),
                                            (64, 1000, torch.float16, 16),
                                            (17, 136, torch.bfloat16, 11)])
def test_gemv_against_float64(R, C, dtype, nvec):
    print(f"gemv {R}x{C} {dtype} nvec={nvec}", flush=True)
    q, masks = structured(R, C, seed=7 * R + C, n_odd=R // 8)
    Q = _q16(q, dtype)
    codes, lut, sal, ex = _k().pack(Q, torch.from_numpy(masks).to(DEV))
    g = torch.Generator().manual_seed(C)
    xf = torch.randn(nvec, C + 24, generator=g)
    x = xf.to(dtype).to(DEV)[:, :C]        # rows strided by C + 24
    y = _k().gemv_packed(codes, lut, sal, C, x, ex)
    torch.cuda.synchronize()
    W64 = Q.double().cpu()
    x64 = x.double().cpu()
    ref = x64 @ W64.t()
    scale = x64.abs() @ W64.abs().t()
    err = (y.double().cpu() - ref).abs()
    assert (err <= 1e-5 * scale + 1e-30).all(), float((err / scale.clamp_min(1e-30)).max())


@pytest.mark.parametrize("R,C,T,dtype", [(37, 300, 17, torch.float16),      # ragged everything
                                          (256, 1024, 64, torch.bfloat16),
                                          (130, 640, 100, torch.float16),
                                          (1000, 4096, 33, torch.bfloat16),   # split K
                                          (300, 2048, 250, torch.float16),
                                          (64, 128, 1, torch.float16)])
def test_gemm_against_float64(R, C, T, dtype):
    """crbq_gemm_packed against float64 products of the unpacked weights,
    same bar as the GEMV; the split-K and single-pass launches are both
    covered (the split depends on R x T tiles)."""
    print(f"gemm {R}x{C} T={T} {dtype}", flush=True)
    from crb_amd import _lib
    q, masks = structured(R, C, seed=5 * R + C, n_odd=R // 8)
    Q = _q16(q, dtype)
    codes, lut, sal, ex = _k().pack(Q, torch.from_numpy(masks).to(DEV))
    g = torch.Generator().manual_seed(T)
    x = torch.randn(T, C + 40, generator=g).to(dtype).to(DEV)[:, :C]
    y = _k().gemm_packed(codes, lut, sal, C, x, ex)
    torch.cuda.synchronize()
    W64 = Q.double().cpu()
    x64 = x.double().cpu()
    ref = x64 @ W64.t()
    scale = x64.abs() @ W64.abs().t()
    err = (y.double().cpu() - ref).abs()
    assert (err <= 1e-5 * scale + 1e-30).all(), float((err / scale.clamp_min(1e-30)).max())
    # the header's rule: floor(512 / tiles) splits of >= 8 blocks each
    tiles = -(-R // 128) * -(-T // (128 if T > 64 else 64))
    split = min(512 // tiles, -(-C // 128) // 8) > 1
    lib = _lib.load()
    assert (lib.crbq_gemm_packed_workspace_size(R, C, T) > 0) == split


def test_gemm_deterministic_and_matches_gemv():
    """Split-K partials are summed in a fixed order: repeated calls are
    bitwise equal; the first 16 tokens agree with the GEMV to the same bar."""
    print("gemm determinism", flush=True)
    q, masks = structured(1000, 4096, seed=9, n_odd=100)
    Q = torch.from_numpy(q).to(DEV)
    codes, lut, sal, ex = _k().pack(Q, torch.from_numpy(masks).to(DEV))
    x = torch.randn(40, 4096, generator=torch.Generator().manual_seed(2)).half().to(DEV)
    y1 = _k().gemm_packed(codes, lut, sal, 4096, x, ex)
    y2 = _k().gemm_packed(codes, lut, sal, 4096, x, ex)
    assert torch.equal(y1, y2)
    yv = _k().gemv_packed(codes, lut, sal, 4096, x[:16], ex)
    scale = x[:16].double().abs() @ Q.double().abs().t()
    assert ((y1[:16].double() - yv.double()).abs() <= 2e-5 * scale + 1e-30).all()


def test_packed_linear_forward():
    print("packed linear", flush=True)
    from crb_amd.packed import PackedLinear
    q, masks = structured(192, 512, seed=11, n_odd=12)
    lin = torch.nn.Linear(512, 192).to(DEV).half()
    lin.weight.data = torch.from_numpy(q).to(DEV)
    pl = PackedLinear.from_linear(lin, torch.from_numpy(masks).to(DEV))
    assert torch.equal(pl.weight(), lin.weight.data)
    assert pl.packed_bytes() * 8 / (192 * 512) < 3.1
    g = torch.Generator().manual_seed(0)
    for ntok in (1, 8, 40, 400):           # 2, 16: GEMV; 80: GEMM; 800: unpack + dense
        x = torch.randn(2, ntok, 512, generator=g).half().to(DEV)
        with torch.no_grad():
            got = pl(x).float()
            want = torch.nn.functional.linear(x.float(), lin.weight.float(), lin.bias.float())
        assert got.shape == (2, ntok, 192)
        assert ((got - want).abs() <= 2e-3 * want.abs() + 2e-3).all(), ntok


def test_stack_pack_option():
    """StackQuantizer(pack=True) leaves PackedLinear modules that decode to
    exactly the weights the unpacked run produces."""
    print("stack pack", flush=True)
    from test_gpu_stack import _samples, tiny_model
    from crb_amd.packed import PackedLinear
    from crb_amd.stack import StackQuantizer, find_linears
    samples = _samples(n=6, seq=96)
    a = tiny_model("opt")
    StackQuantizer(a, chunk=3).run(samples)
    b = tiny_model("opt")
    stats = StackQuantizer(b, chunk=3, pack=True).run(samples)
    assert all(st.packed_bytes > 0 for st in stats)
    for la, lb in zip(a.model.decoder.layers, b.model.decoder.layers):
        dense = find_linears(la)
        for name, m in dense.items():
            mod = lb
            for p in name.split("."):
                mod = getattr(mod, p)
            assert isinstance(mod, PackedLinear), name
            assert torch.equal(mod.weight(), m.weight.data), name
    with torch.no_grad():
        x = samples[:1, :5]
        la_, lb_ = a(x).logits.float(), b(x).logits.float()
    assert torch.allclose(la_, lb_, rtol=2e-2, atol=2e-2)
