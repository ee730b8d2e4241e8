"""CPU replay of the load pipeline of the paired forward kernels
(``born_fwd_fast.h`` and ``born_fwd_d128.h``, function ``top``): Q of the
first item and tiles 0, 1 are issued up front; at the top of step u each wave
waits (``s_waitcnt vmcnt``, loads complete in issue order) until at most
``after`` of its loads are outstanding, the workgroup meets at a barrier, and
then tile u + 2 is issued, plus the second item's Q block at step
``uq = max(1, nt_a - 4)``.  The second item starts at step ``nt_a`` and reads
its Q block from LDS there.

The replay checks, for first items of 1 to 8 tiles and second items of 1 to
10, that every read finds its loads completed before the last barrier, that
the second Q block overwrites the first only after every wave read it, and
that a ring stage is re-filled only after its previous tile's step ended.
Without the drain for short first items (one or two tiles, which the D = 128
purified window launch pairs), the second item's Q block is read before it
has landed: the replay is shown to catch that too.
"""

from __future__ import annotations

import pytest

K_TILE_LOADS = 4  # 1-KiB loads per wave per K + V tile (both kernels: 2 each)
K_Q_LOADS = 8     # 1-KiB loads per wave per Q block
NST = 3


def replay(nt_a: int, ntot: int, purified: bool, drain_short_first: bool = True) -> list[str]:
    """Replays one wave's loads through the pipeline; returns the violations."""
    issued: list[tuple[str, int]] = []  # (name, loads) in issue order
    done = 0  # loads completed (in order)
    visible: set[str] = set()  # groups complete at the last barrier
    bad: list[str] = []
    nitems = 2 if ntot > nt_a else 1
    early_q = nitems == 2
    uq = max(1, nt_a - 4)
    stage_of: dict[int, str] = {}

    def issue(name: str, n: int) -> None:
        issued.append((name, n))

    def outstanding() -> int:
        return sum(n for _, n in issued) - done

    def wait(limit: int) -> None:
        nonlocal done
        while outstanding() > limit:
            done += 1

    def barrier() -> None:
        visible.clear()
        acc = 0
        for name, n in issued:
            acc += n
            if acc <= done:
                visible.add(name)

    def issue_tile(u: int) -> None:
        st = u % NST
        prev = stage_of.get(st)
        # The stage held tile u - 3, read at step u - 3 < u - 2: every wave
        # left that step before the barrier of step u - 2 that issues tile u.
        if prev is not None and int(prev[1:]) != u - NST:
            bad.append(f"stage {st} refilled with T{u} while holding {prev}")
        stage_of[st] = f"T{u}"
        issue(f"T{u}", K_TILE_LOADS)

    issue("Qa", K_Q_LOADS)
    issue_tile(0)
    if ntot > 1:
        issue_tile(1)
    qa_read = False
    for u in range(ntot):
        stores_out = nitems == 2 and u == nt_a + (1 if purified else 2)
        after = 0 if stores_out else ((K_Q_LOADS if (u == uq + 1 and early_q) else 0)
                                      + (K_TILE_LOADS if u + 1 < ntot else 0))
        if after >= K_Q_LOADS + K_TILE_LOADS:
            wait(K_Q_LOADS + K_TILE_LOADS)
        elif after >= K_TILE_LOADS:
            wait(K_TILE_LOADS)
        else:
            wait(0)
        barrier()
        if u == uq and early_q:
            if not qa_read:
                bad.append(f"Qb issued at step {u} before every wave read Qa")
            issue("Qb", K_Q_LOADS)
        if u + 2 < ntot:
            issue_tile(u + 2)
        if drain_short_first and early_q and u == nt_a and nt_a < uq + 2:
            wait(0)
            barrier()
        # Reads of this step.
        if u == 0:
            if "Qa" not in visible:
                bad.append("Qa read before it landed")
        if u == nt_a and nitems == 2 and "Qb" not in visible:
            bad.append(f"Qb read at step {u} before it landed (issued at step {uq})")
        if f"T{u}" not in visible:
            bad.append(f"T{u} read at step {u} before it landed")
        if u == 0:
            qa_read = True  # every wave loads its Q rows at step 0, before the barrier of step 1
    return bad


@pytest.mark.parametrize("purified", [False, True])
@pytest.mark.parametrize("nt_a", range(1, 9))
def test_schedule_every_read_lands(nt_a, purified):
    for nt_b in range(0, 11):
        bad = replay(nt_a, nt_a + nt_b, purified)
        assert not bad, (nt_a, nt_b, bad)


@pytest.mark.parametrize("nt_a", [1, 2])
def test_schedule_replay_catches_short_first_item(nt_a):
    """The pipeline without the drain reads the second Q block early when the
    first item has one or two tiles (what the advisor's replay found)."""
    bad = replay(nt_a, nt_a + 6, purified=True, drain_short_first=False)
    assert any("Qb read" in b for b in bad), bad


@pytest.mark.parametrize("nt_a", range(3, 9))
def test_schedule_drain_only_for_short_first_items(nt_a):
    """From three tiles on, the waits alone cover the second Q block."""
    assert not replay(nt_a, nt_a + 6, purified=True, drain_short_first=False)


def test_d128_window_paired_shapes_have_short_first_items():
    """The GPU regression shapes: B4 H16 with a window, D = 128, on the paired
    purified launch (2 * rounds(pairs) <= rounds(single blocks)): the first
    item (the last query block) has two tiles at T 1800 / W 50 and one at
    T 1850 / W 1."""
    def last_block_tiles(T, W, BM=256, BN=64):
        mb = (T + BM - 1) // BM - 1
        t0 = max(0, mb * BM - W + 1) // BN
        return (min(T, (mb + 1) * BM) + BN - 1) // BN - t0

    def paired(B, H, T):
        nmb = (T + 255) // 256
        npair, nsingle = (nmb + 1) // 2 * B * H, nmb * B * H
        return 2 * ((npair + 255) // 256) <= (nsingle + 255) // 256

    assert paired(4, 16, 1800) and last_block_tiles(1800, 50) == 2
    assert paired(4, 16, 1850) and last_block_tiles(1850, 1) == 1
