"""The fast add-RMSNorm / RMSNorm rows (fp16 rows, 16-byte aligned, h a multiple of
512 up to 4096: every load of a row issued before the first use) against the generic
rows on the same values: the same bits for s, y, rstd, dr, dd and dgamma.  The generic
path is taken by the same data in buffers offset by one element (rows no longer
16-byte aligned), through the C ABI."""

import pytest
import torch

from soupsuck_amd import _lib

pytestmark = pytest.mark.gpu

F16 = _lib.dtype_code(torch.float16)


def placed(src, aligned):
    """src's values in a fresh buffer, 16-byte aligned or offset by one element."""
    flat = torch.empty(src.numel() + 8, device=src.device, dtype=src.dtype)
    off = 0 if aligned else 1
    out = flat[off:off + src.numel()].view(src.shape)
    out.copy_(src)
    return out


def run(device, rows, h, wdt, with_gs, aligned):
    gen = torch.Generator(device="cpu").manual_seed(h + rows)
    r0 = torch.randn((rows, h), generator=gen).half().to(device)
    d0 = torch.randn((rows, h), generator=gen).half().to(device)
    gs0 = torch.randn((rows, h), generator=gen).half().to(device)
    gy0 = torch.randn((rows, h), generator=gen).half().to(device)
    w0 = (1 + 0.1 * torch.randn(h, generator=gen)).to(wdt).to(device)
    r, d, gs, gy, w = (placed(t, aligned) for t in (r0, d0, gs0, gy0, w0))
    wd = _lib.dtype_code(wdt)
    s, y, dr, dd, y1 = (placed(torch.zeros_like(r0), aligned) for _ in range(5))
    rstd = torch.empty(rows, device=device)
    rstd1 = torch.empty(rows, device=device)
    stream = _lib.stream(device)
    _lib.call("ss_add_rmsnorm_fwd", r.data_ptr(), F16, d.data_ptr(), F16, w.data_ptr(), wd, 1,
              s.data_ptr(), F16, y.data_ptr(), F16, rstd.data_ptr(), rows, h, 1e-6, stream)
    _lib.call("ss_rmsnorm_fwd", r.data_ptr(), F16, h, w.data_ptr(), wd, 1, y1.data_ptr(), F16,
              rstd1.data_ptr(), rows, h, 1e-6, stream)
    gsp = gs.data_ptr() if with_gs else None
    _lib.call("ss_add_rmsnorm_bwd", s.data_ptr(), F16, w.data_ptr(), wd, 1, rstd.data_ptr(),
              gsp, F16, h, 1, gy.data_ptr(), F16, h, 1, dr.data_ptr(), F16, dd.data_ptr(), F16,
              rows, h, stream)
    dr2, dd2 = (placed(torch.zeros_like(r0), aligned) for _ in range(2))
    waves = _lib.load().ss_add_rmsnorm_dgamma_waves(rows)
    partial = torch.empty((waves, h), device=device)
    dw = torch.empty(h, device=device, dtype=torch.float16)
    _lib.call("ss_add_rmsnorm_bwd_dgamma", s.data_ptr(), F16, w.data_ptr(), wd, 1,
              rstd.data_ptr(), gsp, F16, h, 1, gy.data_ptr(), F16, h, 1, dr2.data_ptr(), F16,
              dd2.data_ptr(), F16, 1, partial.data_ptr(), dw.data_ptr(), F16, rows, h, stream)
    torch.cuda.synchronize()
    return [t.clone() for t in (s, y, rstd, y1, rstd1, dr, dd, dr2, dd2, dw)]


@pytest.mark.parametrize("rows,h", [(826, 1536), (77, 3584), (130, 512), (5, 4096)])
@pytest.mark.parametrize("wdt", [torch.float16, torch.float32])
@pytest.mark.parametrize("with_gs", [True, False])
def test_fast_rows_match_generic_rows(device, rows, h, wdt, with_gs):
    print(f"case norm rows={rows} h={h} w={wdt} gs={with_gs}", flush=True)
    fast = run(device, rows, h, wdt, with_gs, aligned=True)
    generic = run(device, rows, h, wdt, with_gs, aligned=False)
    names = ("s", "y", "rstd", "rmsnorm y", "rmsnorm rstd", "dr", "dd", "dr (dgamma pass)",
             "dd (dgamma pass)", "dgamma")
    for name, a, b in zip(names, fast, generic):
        assert torch.equal(a, b), name
