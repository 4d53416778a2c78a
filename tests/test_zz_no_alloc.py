"""GPU test of the allocation-free forward split (mxgg_grouped_fwd_split_noalloc)
through the C ABI: bit-identical to mxgg_grouped_fwd_split with a caller
workspace, and within the oracle's GEMM bound, on consecutive calls whose
second input is smaller (the library's scratch keeps the previous call's
contents), then on a call that does not split at all."""
import numpy as np
import pytest
import torch

from mxfp8gg import _lib, ops, workloads
from oracle import oracle as O
from tests._helpers import assert_close_to_oracle, u8

pytestmark = pytest.mark.gpu


def _rand_q(shape, gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    codes = torch.randint(0, 0x7E, shape, generator=g, device=gpu, dtype=torch.int32)
    sign = torch.randint(0, 2, shape, generator=g, device=gpu, dtype=torch.int32) << 7
    s = torch.randint(118, 136, shape[:-1] + (shape[-1] // 32,), generator=g, device=gpu,
                      dtype=torch.int32).to(torch.uint8)
    return (codes | sign).to(torch.uint8), s


def _call(gpu, entry, sizes, N, K, seed, out_dtype=torch.bfloat16):
    E, M = len(sizes), int(np.sum(sizes))
    a, a_s = _rand_q((M, K), gpu, seed)
    w, w_s = _rand_q((E, N, K), gpu, seed + 1)
    ends = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    sa, ldas = ops._scales_2d(a_s, M, K // 32, "a_s")
    sw, wsg, ldws = ops._scales_3d(w_s, E, N, K // 32, "w_s")
    out = torch.full((M, N), float("nan"), dtype=out_dtype, device=gpu)
    lib = _lib.load()
    args = (a.data_ptr(), K, sa.data_ptr(), ldas, w.data_ptr(), N * K, K, sw.data_ptr(), wsg, ldws,
            ends.data_ptr(), E, M, N, K, out.data_ptr(), N, ops._out_code(out_dtype))
    stream = torch.cuda.current_stream(gpu).cuda_stream
    if entry == "noalloc":
        st = lib.mxgg_grouped_fwd_split_noalloc(*args, stream)
    else:
        ws = torch.empty(lib.mxgg_grouped_fwd_workspace_bytes(), dtype=torch.uint8, device=gpu)
        st = lib.mxgg_grouped_fwd_split(*args, ws.data_ptr(), ws.numel(), stream)
    assert st == _lib.OK, lib.mxgg_last_error()
    torch.cuda.synchronize()
    return out, (a, a_s, w, w_s, workloads.ends_of(sizes))


CALLS = [
    ([300, 0, 700, 24], 2048, 4096),     # 8 n-tiles x 6 m-tiles: split ~5 ways
    ([200, 56], 512, 2048),              # smaller: 2 x 2 tiles, split 16 ways
    ([4096, 4096], 4096, 1024),          # 512 tiles: whole rounds, no split
]


def test_noalloc_split_matches_workspace_split_on_consecutive_calls(gpu):
    for i, (sizes, N, K) in enumerate(CALLS):
        print(f"call {i}: sizes {sizes} N {N} K {K}", flush=True)
        got, (a, a_s, w, w_s, ends) = _call(gpu, "noalloc", sizes, N, K, 200 + 3 * i)
        want, _ = _call(gpu, "workspace", sizes, N, K, 200 + 3 * i)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {i}"
        rows = np.unique(np.r_[0, np.cumsum(sizes) - 1, np.arange(0, int(np.sum(sizes)), 97)])
        rows = rows[rows < int(np.sum(sizes))]
        ri = torch.from_numpy(rows).to(gpu)
        assert_close_to_oracle(got[ri], _rows_ref(a, a_s, w, w_s, ends, rows, gpu))


def _rows_ref(a, a_s, w, w_s, ends, rows, gpu):
    gids = np.searchsorted(ends, rows, side="right")
    ri = torch.from_numpy(rows).to(gpu)
    aq, asc = u8(a[ri]), u8(a_s[ri])
    out = np.empty((rows.size, w.shape[1]))
    for g in np.unique(gids):
        sel = gids == g
        out[sel] = O.dequant(aq[sel], asc[sel]) @ O.dequant(u8(w[int(g)]), u8(w_s[int(g)])).T
    return out


def test_noalloc_split_f32_output(gpu):
    got, _ = _call(gpu, "noalloc", [100, 412], 1024, 2048, 300, torch.float32)
    want, _ = _call(gpu, "workspace", [100, 412], 1024, 2048, 300, torch.float32)
    assert torch.equal(got, want)
