"""The Q4_K prefill GEMM's tile plan (qvx_qgemm_plan_q4k), checked on the CPU: every launch's tiles,
decoded the way the kernel decodes its block index, cover each (token, 256-row column) of the
output exactly once, and the K splits cover every 64-element slice once from super-block
boundaries.  A tile lost, doubled or placed past the output would show here before any GPU run."""
import pytest

import qorvix_amd as qvx

SHAPES = [(2048, 14336, 4096), (1024, 14336, 4096), (1025, 14336, 4096), (512, 14336, 4096),
          (128, 14336, 4096), (257, 28672, 4096), (2048, 4096, 14336), (300, 4096, 14336),
          (1536, 14336, 4096), (4096, 14336, 4096), (8192, 4096, 4096), (777, 1000, 4096),
          (64, 256, 256), (1, 128256, 4096), (3000, 6144, 1024), (16384, 28672, 4096)]


def _split_ranges(nsl, splits):
    per = ((nsl + splits - 1) // splits + 3) & ~3
    return [(z * per, min(nsl, z * per + per)) for z in range(splits)]


def _tiles(L, nt):
    """(col, m0) of each block index of one launch: the kernel's XCD-contiguous renumbering, then
    cols_a columns of mt_a tiles from base_a and the rest of mt_b tiles from base_b."""
    nb = L["tiles"]
    order = [(b & 7) * (nb >> 3) + (b >> 3) if nb % 8 == 0 else b for b in range(nb)]
    assert sorted(order) == list(range(nb)), "renumbering is not a permutation"
    na = L["cols_a"] * L["mt_a"]
    out = []
    for b in order:
        if b < na:
            out.append((b // L["mt_a"], L["base_a"] + (b % L["mt_a"]) * L["bm"]))
        else:
            b -= na
            out.append((L["cols_a"] + b // L["mt_b"], L["base_b"] + (b % L["mt_b"]) * L["bm"]))
    return out


@pytest.mark.parametrize("cus", [256, 304, 80, 32])
@pytest.mark.parametrize("M,rows,cols", SHAPES)
def test_plan_covers_output_once(M, rows, cols, cus):
    plan = qvx.qgemm_plan_q4k(M, rows, cols, cus)
    assert 1 <= len(plan) <= 2
    nt = (rows + 255) // 256
    nsl = cols // 64
    cover = [[0] * M for _ in range(nt)]
    for L in plan:
        assert L["bm"] in (128, 192, 256) and L["splits"] >= 1
        splits = _split_ranges(nsl, L["splits"])
        assert [a for a, _ in splits] == [4 * (a // 4) for a, _ in splits]
        assert sorted(k for a, b in splits for k in range(a, b)) == list(range(nsl))
        for col, m0 in _tiles(L, nt):
            assert 0 <= col < nt and m0 >= 0
            for m in range(m0, min(M, m0 + L["bm"])):
                cover[col][m] += 1
        if len(plan) == 2:
            assert L["splits"] == 1  # two-launch plans never split K
    assert all(c == 1 for row in cover for c in row)


def test_balanced_plan_for_config4():
    """2048 x 14336 on 256 CUs: one full round of 256-token tiles, one of 192-token tiles."""
    plan = qvx.qgemm_plan_q4k(2048, 14336, 4096, 256)
    assert [(L["bm"], L["tiles"]) for L in plan] == [(256, 256), (192, 256)]


def test_plan_rejections():
    assert qvx.lib().qvx_qgemm_plan_q4k(0, 256, 256, 0, None, 0) == qvx.E_SHAPE
    assert qvx.lib().qvx_qgemm_plan_q4k(16, 256, 100, 0, None, 0) == qvx.E_SHAPE
