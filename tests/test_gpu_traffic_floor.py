"""The schedule's traffic floor (vcsrmc_traffic_floor) against a count made here from the CSR:
each unit's row part follows the dealing rule of the launch (heavy unit u to part u mod parts,
light unit num_heavy + j to the part whose xcd_start range holds j), a part's B bytes are the
distinct columns of its units' rows times O times the element size, C the non-empty rows, and
the layout's bytes per O tile follow from the counts of units, tiles and entries."""
import numpy as np
import pytest

import vcsr_mc_amd as vm
from conftest import random_csr
from gpu_util import dev, say

pytestmark = pytest.mark.gpu

SPLIT, ROW_STEPS = 1 << 16, 1 << 18


def parts_of_units(units, xcd_start, num_heavy, row_parts):
    G = 8 // row_parts
    part = np.empty(len(units), np.int64)
    part[:num_heavy] = np.arange(num_heavy) % row_parts
    j = np.arange(len(units) - num_heavy)
    bounds = np.array([xcd_start[(r + 1) * G] for r in range(row_parts - 1)], np.int64)
    part[num_heavy:] = np.searchsorted(bounds, j, side="right")
    return part


@pytest.mark.parametrize("fp32", [False, True])
@pytest.mark.parametrize("O,tileK", [(128, 128), (256, 128), (100, 32), (64, 64)])
def test_floor_matches_csr_count(fp32, O, tileK):
    rng = np.random.default_rng(O + tileK + fp32)
    M, N = 5000, 7000
    rp, c, v = random_csr(rng, M, N, density=0.002, empty_frac=0.1)
    say("traffic floor", fp32, O, tileK, M, N, c.size)
    vm.set_fp32_row_steps(0)
    try:
        with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, fp32, 32) as f:
            info = f.info()
            assert info["num_split_panels"] == 0 and info["num_dense"] == 0
            units, xs = f.units()
            rows = f.rows_of_units(units)
            for overwrite in (False, True):
                t = f.traffic_floor(O, tileK=tileK, b_f16=not fp32, overwrite=overwrite)
                part = parts_of_units(units, xs, info["num_heavy"], t["row_parts"])
                seen = np.zeros((t["row_parts"], N), bool)
                for u, rr in enumerate(rows):
                    cols = np.concatenate([c[rp[r]:rp[r + 1]] for r in rr]) if rr.size else []
                    seen[part[u], cols] = True
                sb = 4 if fp32 else 2
                assert t["b_bytes"] == int(seen.sum()) * O * sb
                assert t["b_once_bytes"] == int(seen.any(axis=0).sum()) * O * sb
                ne = int(np.count_nonzero(np.diff(rp)))
                assert t["c_bytes"] == ne * O * 4 * (1 if overwrite else 2)
                per_tile = 8 + 128
                a = 16 * info["num_units"] + per_tile * info["num_chunks"] + \
                    c.size * (8 if fp32 else 4)
                assert t["o_tiles"] == -(-O // t["o_tile_width"])
                assert t["a_bytes"] == a * t["o_tiles"]
                assert t["total"] == t["b_bytes"] + t["a_bytes"] + t["c_bytes"] + \
                    t["convert_bytes"] and t["convert_bytes"] == 0
    finally:
        vm.set_fp32_row_steps(1)


def test_floor_counts_split_panels_and_row_steps(orc):
    """Heavy rows (split panels, counted once at their first unit) and FP32 row-step batches
    (640 bytes each: column slots and the values the lanes read)."""
    rng = np.random.default_rng(5)
    M, N = 3000, 40000
    rp, c, v = random_csr(rng, M, N, density=0.0004, heavy_rows=3, heavy_nnz=30000,
                          empty_frac=0.2)
    say("traffic floor: split panels and row steps", c.size)
    vm.set_fp32_row_steps(2)
    try:
        with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, True, 32) as f:
            info = f.info()
            assert info["num_split_panels"] > 0
            units, _ = f.units()
            t = f.traffic_floor(64, tileK=64)
            ne = int(np.count_nonzero(np.diff(rp)))
            assert t["c_bytes"] == ne * 64 * 4 * 2
            rs = (units[:, 3] & ROW_STEPS) != 0
            batches = int((units[rs, 2] - units[rs, 1]).sum())
            assert batches == info["num_row_step_batches"] > 0
            assert t["a_bytes"] >= (16 * info["num_units"] + 640 * batches) * t["o_tiles"]
    finally:
        vm.set_fp32_row_steps(1)


def test_floor_and_units_edge_cases():
    """An empty matrix has no units and a zero floor; a bad tileK and FP16 B for an FP32 format
    are refused with the launch's own errors; units of a 3-row matrix cover its rows."""
    import torch
    rp = np.zeros(6, np.int32)
    say("traffic floor: edge cases")
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(np.zeros(0, np.int32)),
                                         dev(np.zeros(0, np.float32)), 5, 7, False, 32) as f:
        units, xs = f.units()
        assert units.shape == (0, 4) and xs.tolist() == [0] * 9
        t = f.traffic_floor(128)
        assert t["total"] == 0 and t["b_bytes"] == 0 and t["c_bytes"] == 0
    rp = np.array([0, 2, 2, 5], np.int32)
    c = np.array([0, 9, 1, 2, 9], np.int32)
    v = np.ones(5, np.float32)
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), 3, 10, True, 32) as f:
        units, _ = f.units()
        rows = np.unique(np.concatenate(f.rows_of_units(units)))
        assert rows.tolist() == [0, 2]  # row 1 holds no nonzero
        with pytest.raises(vm.VCSRMCError) as e:
            f.traffic_floor(64, tileK=48)
        assert e.value.status == vm.ERR_TILEK
        with pytest.raises(vm.VCSRMCError) as e:
            f.traffic_floor(64, b_f16=True)
        assert e.value.status == vm.ERR_ARG
        t = f.traffic_floor(64)
        # four distinct columns, FP32 B, one row part holding them all, two rows of C
        assert t["b_once_bytes"] == 4 * 64 * 4 and t["c_bytes"] == 2 * 64 * 4 * 2
