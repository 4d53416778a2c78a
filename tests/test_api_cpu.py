"""Host-side logic that runs without a GPU: reference-named modules import,
argument handling fails loudly on CPU tensors (no CPU fallback), offs
normalisation, and the torchao swap-in against a fake torchao module."""
import sys
import types

import numpy as np
import pytest
import torch

import fused_fwd
import fwd_final
import mxfp8gg
import patch_kernels
import wgrad_fused
from mxfp8gg import ops, workloads


def test_reference_module_names_resolve():
    assert fused_fwd.fused_grouped_fwd is mxfp8gg.fused_grouped_fwd
    assert fwd_final.fwd_ge is mxfp8gg.fwd_ge
    assert wgrad_fused.wgrad_fused is mxfp8gg.wgrad_fused
    assert wgrad_fused.wgrad_prepare is mxfp8gg.wgrad_prepare
    assert wgrad_fused.wgrad_kernel is mxfp8gg.wgrad_kernel
    assert callable(patch_kernels.apply)


def test_best_config_matches_reference_heuristic():
    # wgrad_fused.py:22-31
    assert wgrad_fused._best_config(8, 128000)["BLOCK_M"] == 256
    assert wgrad_fused._best_config(4, 32768)["num_stages"] == 2
    assert wgrad_fused._best_config(8, 32768)["num_stages"] is None


def test_cpu_tensors_are_rejected_not_computed():
    a = torch.zeros(64, 256, dtype=torch.float8_e4m3fn)
    w = torch.zeros(2, 32, 256, dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="ROCm GPU only"):
        fused_fwd.fused_grouped_fwd(a, w, torch.tensor([32, 64], dtype=torch.int32))
    with pytest.raises(ValueError, match="ROCm GPU only"):
        mxfp8gg.to_mxfp8_dim0(torch.zeros(4, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="ROCm GPU only"):
        mxfp8gg.wgrad_fused(torch.zeros(8, 64, dtype=torch.float8_e4m3fn),
                            torch.zeros(8, 64, dtype=torch.float8_e4m3fn),
                            torch.tensor([64], dtype=torch.int32))


def test_offs_forms():
    dev = torch.device("cpu")
    ends = ops._group_ends(torch.tensor([0, 3, 7, 9], dtype=torch.int32), 3, dev)
    assert ends.tolist() == [3, 7, 9]
    ends = ops._group_ends(torch.tensor([3, 7, 9], dtype=torch.int64), 3, dev)
    assert ends.dtype == torch.int32 and ends.tolist() == [3, 7, 9]
    with pytest.raises(ValueError):
        ops._group_ends(torch.tensor([1, 2]), 3, dev)


def test_padded_capacity():
    assert ops.padded_token_capacity(64, None) == 64
    assert ops.padded_token_capacity(65, None) == 96
    assert ops.padded_token_capacity(100, 4) == 256   # 100 + 4*31 rounded up to 128
    assert ops.padded_token_capacity(65536, 32) % 128 == 0


def test_workload_routing_shapes():
    s2 = workloads.dirichlet_sizes(65536, 32, 0)
    assert s2.sum() == 65536 and s2.shape == (32,)
    s4 = workloads.zipf_sizes(65536, 32, 1.2, 0, empty=2)
    assert s4.sum() == 65536 and (s4 == 0).sum() >= 2 and s4.max() > 16384
    assert workloads.ends_of([1, 0, 2]).tolist() == [1, 1, 3]


def test_apply_patches_a_fake_torchao(monkeypatch):
    names = ["torchao", "torchao.prototype", "torchao.prototype.moe_training",
             "torchao.prototype.moe_training.kernels",
             "torchao.prototype.moe_training.kernels.mxfp8",
             "torchao.prototype.moe_training.kernels.mxfp8.rocm_mxfp8_mm",
             "torchao.prototype.moe_training.kernels.mxfp8.quant"]
    for n in names:
        monkeypatch.setitem(sys.modules, n, types.ModuleType(n))
    target = sys.modules[names[5]]
    target.triton_mxfp8_grouped_mm = object()
    patch_kernels.apply()
    assert target.triton_mxfp8_grouped_mm is mxfp8gg.triton_mxfp8_grouped_mm
    assert target.triton_mxfp8_wgrad is mxfp8gg.triton_mxfp8_wgrad
    assert target.triton_mxfp8_wgrad_v2 is mxfp8gg.triton_mxfp8_wgrad
    assert sys.modules[names[4]].rocm_mxfp8_mm is target
    assert sys.modules[names[6]].triton_to_mxfp8_dim0 is mxfp8gg.triton_to_mxfp8_dim0


def test_apply_without_torchao_raises():
    if "torchao" in sys.modules:
        pytest.skip("torchao importable here")
    with pytest.raises(ImportError):
        patch_kernels.apply()


def test_forward_rows_per_launch_stay_under_the_buffer_range():
    # one launch reads A through a 32-bit buffer range: (rows - 1) * lda + K
    # must stay below 0x7FFFFFF0; larger A runs in chunks of whole 256-row tiles
    assert ops._rows_per_launch(7168, 7168, 1000) == 1000
    assert ops._rows_per_launch(7168, 7168, 0) == 1
    r = ops._rows_per_launch(7168, 7168, 360000)
    assert r == 299520 and r % 256 == 0 and (r - 1) * 7168 + 7168 <= 0x7FFFFFF0
    assert (r + 256 - 1) * 7168 + 7168 > 0x7FFFFFF0      # the next multiple would not fit
    lda = 1 << 23   # the largest row stride the C ABI accepts
    assert ops._rows_per_launch(lda, 4096, 1000) == 256


def test_wgrad_split_choice():
    # enough tiles for every compute unit: no split
    assert ops.wgrad_split_tokens(65536, 4096, 7168, 32, 256) == 0
    # 128 tiles on 256 units: 2 chunks per expert fill the other half
    assert ops.wgrad_split_tokens(65536, 2048, 1024, 4, 256) == 8192
    # 512 tiles: the partials would cost more than the idle units
    assert ops.wgrad_split_tokens(65536, 2048, 2048, 8, 256) == 0
    # 8 tiles: at most 16 chunks, none shorter than 4096 tokens
    assert ops.wgrad_split_tokens(131072, 512, 512, 2, 256) == 4096
    # 2 experts x 4 x 4 tiles = 32 on 256 units: 8 chunks of 4096 tokens
    assert ops.wgrad_split_tokens(65536, 1024, 1024, 2, 256) == 4096
    # 1 expert x 8 x 8 tiles = 64: 4 chunks
    assert ops.wgrad_split_tokens(32768, 2048, 2048, 1, 256) == 8192
    # short groups are not split below 4096 tokens
    assert ops.wgrad_split_tokens(4096, 256, 256, 2, 256) == 0


def test_forward_split_entry_choice(monkeypatch):
    # a workspace of 256 partials: a round is 256 tiles
    monkeypatch.setattr(ops, "_split_workspace_bytes", lambda device: 16384 + 256 * 256 * 4 * 256)
    # one expert over exactly 16 rounds: no last round to cut, no reduce launch
    assert not ops._full_rounds(65536, 4096, 1, None)
    assert not ops._small_launch(65536, 4096, 1, None)
    # one more m-tile: a last round of 16 tiles, cut along K
    assert ops._full_rounds(65536 + 1, 4096, 1, None)
    # 32 ragged experts (C2): 256..287 m-tiles, some counts leave <= 128 tiles
    assert ops._full_rounds(65536, 4096, 32, None)
    # 5 experts over 6400 rows: 25..30 m-tiles x 16 n-tiles = 400..480 tiles,
    # a last round of 144..224 tiles whatever the sizes: no split entry
    assert not ops._full_rounds(6400, 4096, 5, None)
    # 8 experts: up to 33 m-tiles, and 528 tiles leave a last round of 16
    assert ops._full_rounds(6400, 4096, 8, None)
    # less than a round: the small-launch rule decides
    assert not ops._full_rounds(512, 2048, 1, None)
    assert ops._small_launch(512, 2048, 1, None)


# ---------------------------------------------------------------------------
# weight-cast cache (host logic only: a stub stands in for the GPU cast)
# ---------------------------------------------------------------------------
def _stub_cache(max_entries=4):
    from mxfp8gg.weight_cache import WeightCastCache
    calls = []

    def cast(w, mode):
        calls.append((id(w), w._version, mode))
        return (("q", len(calls)), ("t", len(calls)))

    return WeightCastCache(max_entries=max_entries, cast=cast), calls


def test_weight_cache_hits_until_the_weight_changes():
    cache, calls = _stub_cache()
    w = torch.zeros(2, 32, 64)
    a = cache.get(w, "rceil")
    assert cache.get(w, "rceil") is a and len(calls) == 1 and cache.hits == 1
    w.add_(1.0)                                   # in-place update bumps the version
    b = cache.get(w, "rceil")
    assert b is not a and len(calls) == 2
    assert len(cache) == 1                         # the stale entry was dropped
    cache.get(w, "floor")                          # the scale mode is part of the key
    assert len(calls) == 3


def test_weight_cache_distinguishes_tensors_and_evicts_lru():
    cache, calls = _stub_cache(max_entries=2)
    ws = [torch.zeros(1, 32, 32) for _ in range(3)]
    for w in ws:
        cache.get(w)
    assert len(calls) == 3 and len(cache) == 2     # the oldest entry was evicted
    cache.get(ws[2])
    assert len(calls) == 3                          # still cached
    cache.get(ws[0])
    assert len(calls) == 4                          # evicted earlier, cast again
    cache.clear()
    assert len(cache) == 0


def test_bench_refuses_more_than_one_gpu():
    # one GPU's expert share is the measured unit: --gpus 2 exits with a message
    # before touching a device
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_offs_helpers_reject_cpu_tensors():
    t = torch.tensor([4, 4], dtype=torch.int32)
    with pytest.raises(ValueError, match="ROCm GPU only"):
        mxfp8gg.offs_to_group_ends(t, 8)
    with pytest.raises(ValueError, match="offs_kind"):
        mxfp8gg.offs_to_group_ends(t, 8, "cumulative")
    with pytest.raises(ValueError, match="ROCm GPU only"):
        mxfp8gg.zero_rows_past_groups(torch.zeros(4, 8), t)


def test_group_ends_type_survives_copies_only():
    t = ops._mark_ends(torch.tensor([64, 64, 64, 64], dtype=torch.int32))
    assert isinstance(t, mxfp8gg.GroupEnds)
    import copy
    kept = [t.clone(), t.detach(), t.to(torch.int64), t.cpu(), t.contiguous(), t.int(),
            copy.deepcopy(t), torch.cat([t, t.clone()]), torch.stack([t, t])]
    assert all(isinstance(k, mxfp8gg.GroupEnds) for k in kept)
    assert all(k.flatten()[:4].tolist() == [64, 64, 64, 64] for k in kept)
    # arithmetic, indexing and mixed concatenation give plain tensors
    dropped = [t + 1, t[1:], t.diff(), torch.cat([t, torch.tensor([1], dtype=torch.int32)])]
    assert not any(isinstance(d, mxfp8gg.GroupEnds) for d in dropped)


def test_ambiguous_offs_warning_is_opt_in(monkeypatch):
    import warnings

    amb = torch.tensor([64, 64, 64, 64], dtype=torch.int32)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        monkeypatch.delenv("MXGG_CHECK_OFFS", raising=False)
        ops._warn_if_ambiguous(amb, 256)                 # off by default
        monkeypatch.setenv("MXGG_CHECK_OFFS", "1")
        ops._warn_if_ambiguous(torch.tensor([64, 128, 192, 256]), 256)   # ends only
        ops._warn_if_ambiguous(torch.tensor([100, 50, 106]), 256)        # sizes only
        with pytest.raises(RuntimeWarning, match="reads as group sizes and as cumulative"):
            ops._warn_if_ambiguous(amb, 256)
