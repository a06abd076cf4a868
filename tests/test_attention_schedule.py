"""CPU model of fa_fwd2's per-wave schedule (autokernel_amd/csrc/attention.hip): barriers, K / V
LDS-DMA transfers and LDS stage reads, for the 4-wave blocks (NH = 1) and the 8-wave blocks that
split the key tiles over two wave groups (NH = 2). No GPU: the model restates the kernel's issue /
wait / read sequence (attention.hip:496 the per-wave last tile, :643-662 barrier_after / sync_mid /
sync_end, :664-740 the general and steady iterations, :753-785 the prologue and the iteration loop,
:787 the hand-over between the halves) and checks, for every wave of every block:
  * all waves of a block execute the same number of s_barrier (a mismatch would hang the block);
  * every transfer targets a key tile of the block (its buffer resource starts at or before the
    last key);
  * every read of a stage finds the expected tile, and each of the four waves of that half had
    waited for its own transfers of the tile before a barrier that precedes the read;
  * no transfer refills a stage before the barrier that follows every read of its previous tile;
  * no transfer is outstanding when a wave leaves the loop.
Planted mistakes (an uncapped per-wave last tile, the second half iterating its own tile count, one
K tile too many) must be caught, so the checks are not vacuous."""
import pytest

BKV, BQ, WAVES = 64, 128, 4


def wave_events(nt, ntl, jw, jf, nh, k_extra=0):
    """One wave's events: ('issue', mat, tile, stage), ('wait', newest groups allowed in flight),
    ('bar',), ('read', mat, stage, tile). Tiles are relative to the half's first tile."""
    ev = []

    def issue(mat, j, stage):
        ev.append(("issue", mat, j, stage))

    def barrier_after(later):
        ev.append(("wait", 2 if later >= 2 else (1 if later == 1 else 0)))
        ev.append(("bar",))

    def sync_mid(j, par):
        barrier_after(int(nt > 2) if j == 0 else 1 + int(j + 2 < nt))
        if j + 1 < nt:
            issue("V", j + 1, par ^ 1)

    def sync_end(j, par):
        barrier_after(int(j + 2 < nt) + int(j + 1 < nt))
        if j + 3 < nt + k_extra:  # k_extra = 1: a planted mistake
            issue("K", j + 3, par ^ 1)

    def general(j, par):
        if j > 0 and j - 1 <= jw:
            ev.append(("read", "V", par ^ 1, j - 1))
        sync_mid(j, par)
        if j + 1 <= jw:
            ev.append(("read", "K", par ^ 1, j + 1))
        sync_end(j, par)

    def steady(j, par):
        ev.append(("read", "V", par ^ 1, j - 1))
        sync_mid(j, par)
        ev.append(("read", "K", par ^ 1, j + 1))
        sync_end(j, par)

    issue("K", 0, 0)
    if nt > 1:
        issue("K", 1, 1)
    issue("V", 0, 0)
    ev += [("wait", 0), ("bar",), ("read", "K", 0, 0), ("wait", 0), ("bar",)]
    if nt > 2:
        issue("K", 2, 0)
    general(0, 0)
    j = 1
    while j + 1 < jf:
        steady(j, 1)
        steady(j + 1, 0)
        j += 2
    if j < jf:
        steady(j, 1)
        j += 1
    while j < ntl:
        general(j, j & 1)
        j += 1
    if ntl - 1 <= jw:
        ev.append(("read", "V", (ntl - 1) & 1, ntl - 1))
    ev.append(("wait", 0))
    if nh == 2:
        ev += [("wait", 0), ("bar",), ("bar",)]
    return ev


def block_waves(Sq, Sk, causal, qb, nh, cap_jw=True, second_half_own_count=False, k_extra=0):
    q0 = qb * BQ
    kend = min(Sk, q0 + BQ) if causal else Sk
    ntb = (kend + BKV - 1) // BKV
    ntl = (ntb + 1) // 2 if nh == 2 else ntb
    out = []
    for half in range(nh):
        jbase = half * ntl
        nt = (ntb - ntl if half else ntl) if nh == 2 else ntb
        assert nt >= 1
        for w in range(WAVES):
            qw0 = q0 + w * 32
            last = (min(ntb - 1, (qw0 + 31) // BKV) if causal else ntb - 1) - jbase
            jw = min(nt - 1, last) if cap_jw else last
            jm_s = Sk // BKV - jbase
            jm = min((qw0 + 1) // BKV - jbase, jm_s) if causal else jm_s
            jf = max(1, min(jm, jw))
            loop = nt if second_half_own_count else ntl
            out.append((half, w, nt, wave_events(nt, loop, jw, jf, nh, k_extra)))
    return out


def check_block(waves, nh):
    nbar = {sum(1 for e in ev if e[0] == "bar") for (_, _, _, ev) in waves}
    assert len(nbar) == 1, ("barrier counts differ", sorted(nbar))
    for half in range(nh):
        hw = [x for x in waves if x[0] == half]
        landed, issued = {}, {}
        for (_, w, nt, ev) in hw:
            pending, nb = [], 0
            for e in ev:
                if e[0] == "issue":
                    assert 0 <= e[2] < nt, ("transfer past the block's keys", e, nt)
                    pending.append((e[1], e[2]))
                    issued[(e[1], e[2], w)] = nb
                elif e[0] == "wait":
                    keep = e[1]
                    done, pending = (pending[:-keep], pending[-keep:]) if keep else (pending, [])
                    for g in done:
                        landed[(g, w)] = nb + 1
                elif e[0] == "bar":
                    nb += 1
            assert not pending, ("transfers outstanding at the end", pending)
        for (_, w, nt, ev) in hw:
            nb = 0
            for e in ev:
                if e[0] == "bar":
                    nb += 1
                elif e[0] == "read":
                    mat, stage, j = e[1], e[2], e[3]
                    assert j % 2 == stage, ("stage parity", e)
                    for w2 in range(WAVES):
                        lb = landed.get(((mat, j), w2))
                        assert lb is not None and lb <= nb, ("read before the tile landed", e, w2, lb, nb)
                        nxt = issued.get((mat, j + 2, w2))
                        assert nxt is None or nxt > nb, ("stage refilled before its read", e, w2, nxt, nb)


def _cases(nh):
    sks = list(range(256 if nh == 2 else 64, 900, 7)) + [1024, 2048, 8192]
    for causal in (0, 1):
        for Sk in sks:
            for Sq in ([Sk, Sk // 2 + 1, Sk + 37] if causal else [Sk]):
                for qb in range(-(-Sq // BQ)):
                    yield Sq, Sk, causal, qb


@pytest.mark.parametrize("nh", [1, 2])
def test_schedule(nh):
    n = 0
    for Sq, Sk, causal, qb in _cases(nh):
        check_block(block_waves(Sq, Sk, causal, qb, nh), nh)
        n += 1
    assert n > 1000


@pytest.mark.parametrize("plant", ["uncapped last tile", "second half iterates its own count", "one K tile too many"])
def test_planted_mistakes_are_caught(plant):
    kw = {"uncapped last tile": dict(cap_jw=False), "second half iterates its own count": dict(second_half_own_count=True),
          "one K tile too many": dict(k_extra=1)}[plant]
    with pytest.raises(AssertionError):
        for Sq, Sk, causal, qb in _cases(2):
            check_block(block_waves(Sq, Sk, causal, qb, 2, **kw), 2)
