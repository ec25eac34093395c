"""GPU frame-deduplicating replay ring (the reference's FrameReplay, src/fast_mario_env/replay.py).

CPU: the numpy oracle (oracle/replay_oracle.py) is pinned against the transitions as they were added:
every sampleable slot rebuilds the stored obs / next_obs stacks, the action, m, the terminal flag, and the
n-step return and discount of a float64 brute-force sum, over episodes with resets, terminations,
truncations, ring wrap-around and ages past 255. GPU: mh_replay_add / mh_replay_gather against the oracle
bit for bit (storage after every add, sampled batches), and the reference's own test, test_replay.py:13-55,
on HipVecEnv transitions."""
import os
import sys

import numpy as np
import pytest

from conftest import requires_gpu, scaled

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
from replay_oracle import ReplayOracle  # noqa: E402


def _episodes(E, k, hw, steps, seed, p_done=0.12, p_trunc=0.35, long_env=None):
    """Synthetic frame-stacked transitions (obs, next_obs, action, reward, done, truncated, terminated) with
    FrameStack semantics: a reset stack is [0, ..., 0, frame]; next_obs of a finished env is its terminal
    stack. `long_env` never finishes (ages saturate)."""
    rng = np.random.default_rng(seed)
    cur = np.zeros((E, k, *hw), np.uint8)
    cur[:, -1] = rng.integers(0, 256, (E, *hw))
    for _ in range(steps):
        f = rng.integers(0, 256, (E, *hw), dtype=np.uint8)
        nxt = np.concatenate([cur[:, 1:], f[:, None]], 1)
        done = rng.random(E) < p_done
        if long_env is not None:
            done[long_env] = False
        trunc = done & (rng.random(E) < p_trunc)
        a = rng.integers(-3, 9, E)                       # out-of-range actions wrap like the int16 store
        r = rng.normal(0, 5, E).astype(np.float32)
        yield cur.copy(), nxt.copy(), a, r, done, trunc, done & ~trunc
        cur = nxt
        for e in np.flatnonzero(done):
            cur[e] = 0
            cur[e, -1] = rng.integers(0, 256, hw)


def _brute(gt, e, p, ns, gamma):
    o, a = gt[(e, p)][:2]
    R, q, term, m, last = 0.0, p, False, 0, None
    for i in range(ns):
        _, _, r, nx, d, te = gt[(e, q)]
        R += gamma ** i * r
        m += 1
        last, term = nx, te
        if d:
            break
        q += 1
    return o, a, R, m, last, term


def _fill(rb_list, E, k, hw, steps, seed, **kw):
    gt = {}
    for obs, nxt, a, r, d, tr, te in _episodes(E, k, hw, steps, seed, **kw):
        for rb in rb_list:
            rb.add(obs, nxt, a, r, d, tr)
        ptr = rb_list[0].ptr
        for e in range(E):
            gt[(e, int(ptr[e]) - 2)] = (obs[e], int(np.int64(a[e]).astype(np.int16)), float(r[e]), nxt[e], bool(d[e]), bool(te[e]))
    return gt


@pytest.mark.parametrize("C,steps,long_env", [(40, 30, None), (13, 90, None), (9, 600, 1)])
def test_oracle_rebuilds_the_added_transitions(C, steps, long_env):
    E, k, hw, gamma = 3, 4, (4, 8), 0.9
    rb = ReplayOracle(C, E, k, hw)
    gt = _fill([rb], E, k, hw, steps, seed=C, long_env=long_env)
    if long_env is not None:
        assert rb.age[long_env].max() == 255             # the age saturates
    for ns in (1, 3):
        pairs = rb.sampleable(ns)
        assert pairs
        out = rb.assemble([e for e, _ in pairs], [p for _, p in pairs], ns, gamma)
        for b, (e, p) in enumerate(pairs):
            o, a, R, m, last, term = _brute(gt, e, p, ns, gamma)
            assert np.array_equal(out["obs"][b], o), (e, p)
            assert out["action"][b] == a and out["steps"][b] == m and bool(out["terminal"][b]) == term
            assert np.array_equal(out["next_obs"][b], last), (e, p, m)
            assert abs(float(out["reward"][b]) - R) < 1e-4 * max(1.0, abs(R))
            assert abs(float(out["discount"][b]) - (0.0 if term else gamma ** m)) < 1e-6


def test_oracle_sampleable_window():
    """Only slots whose k-1 predecessors are still in the ring and whose n-step successors are written, and
    never a terminal frame's slot (those carry no transition)."""
    E, k, hw, C = 2, 4, (4, 4), 11
    rb = ReplayOracle(C, E, k, hw)
    _fill([rb], E, k, hw, 50, seed=3)
    for ns in (1, 2, 5):
        for e, p in rb.sampleable(ns):
            assert rb.ptr[e] - C + k - 1 <= p <= rb.ptr[e] - 1 - ns and rb.flags[e, p % C] & 1


# ---------------------------------------------------------------------------------------------- GPU

def _gpu_state(rb):
    return {n: getattr(rb, n).cpu().numpy() for n in ("frames", "age", "act", "rew", "flags")}


@pytest.mark.gpu
@requires_gpu
@pytest.mark.parametrize("C,steps", [(23, 70), (200, 40)])
def test_replay_kernels_match_oracle(C, steps):
    import torch
    from fast_mario_env_amd.replay import FrameReplay

    E, k, hw = 5, 4, (84, 84)
    gpu = FrameReplay(C, E, k, hw, device="cuda", seed=1)
    orc = ReplayOracle(C, E, k, hw)
    for t, (obs, nxt, a, r, d, tr, _) in enumerate(_episodes(E, k, hw, steps, seed=C)):
        # device tensors for the GPU ring (torch inputs), numpy for the oracle
        gpu.add(torch.from_numpy(obs).cuda(), torch.from_numpy(nxt).cuda(), torch.from_numpy(a).cuda(),
                torch.from_numpy(r).cuda(), torch.from_numpy(d).cuda(), torch.from_numpy(tr).cuda())
        orc.add(obs, nxt, a, r, d, tr)
        if t % 7 == 0 or t == steps - 1:
            g = _gpu_state(gpu)
            for n, v in g.items():
                assert np.array_equal(v, getattr(orc, n)), (n, t)
            assert np.array_equal(gpu.ptr, orc.ptr) and np.array_equal(gpu.new_ep, orc.new_ep)
    for ns, gamma in ((1, 0.99), (3, 0.9)):
        b = gpu.sample(256, ns, gamma)
        env, pos = b.env.cpu().numpy(), b.pos.cpu().numpy()
        ok = set(orc.sampleable(ns))
        assert all((int(e), int(p)) in ok for e, p in zip(env, pos))
        ref = orc.assemble(env, pos, ns, gamma)
        for n in ("obs", "next_obs", "action", "reward", "discount", "terminal", "steps"):
            got = getattr(b, n).cpu().numpy()
            assert got.dtype == ref[n].dtype and np.array_equal(got, ref[n]), (n, ns)
    gpu.check_errors()


@pytest.mark.gpu
@requires_gpu
def test_replay_gather_flags_bad_pairs():
    import torch
    from fast_mario_env_amd.replay import FrameReplay

    rb = FrameReplay(8, 2, 4, (16, 16), device="cuda", seed=0)
    b = rb.gather(torch.tensor([0, 2, 1], device="cuda"), torch.tensor([3, 0, -1], device="cuda"), 2, 0.9)
    assert int(b.obs[1].sum()) == 0 and int(b.next_obs[2].sum()) == 0
    with pytest.raises(IndexError):
        rb.check_errors()
    rb.check_errors()                                    # the flag was cleared


@pytest.mark.gpu
@requires_gpu
def test_replay_exact_on_env_transitions():
    """The reference's test_replay_exact (test_replay.py:13-55) on HipVecEnv transitions."""
    import torch
    from build_roms import rom_path
    from fast_mario_env_amd import HipVecEnv
    from fast_mario_env_amd.replay import FrameReplay

    n, steps, cap, n_step, gamma = 4, scaled(300), 120, 3, 0.9
    v = HipVecEnv("1-1", n, seed=3, max_steps=40, sticky=0.25, noop_max=5, rom=open(rom_path("vanilla"), "rb").read())
    rb = FrameReplay(cap, n, 4, device="cuda", seed=0)
    obs = v.reset().clone()
    g = torch.Generator(device="cuda"); g.manual_seed(0)
    gt = {}
    for _ in range(steps):
        a = torch.randint(0, 7, (n,), generator=g, device="cuda")
        o2, r, te, tr, _ = v.step(a)
        d = te | tr
        nxt = torch.where(d[:, None, None, None], v.final_obs, o2)
        rb.add(obs, nxt, a, r, d, tr & ~te)
        ptr = rb.ptr
        on, nn, an, rn, dn, ten = (x.cpu().numpy() for x in (obs, nxt, a, r, d, te))
        for i in range(n):
            gt[(i, int(ptr[i]) - 2)] = (on[i], int(an[i]), float(rn[i]), nn[i], bool(dn[i]), bool(ten[i]))
        obs = o2.clone()
    v.close()
    assert rb.ptr.min() > cap                            # the ring wrapped around
    bad = checked = 0
    for ns in (1, n_step):
        for _ in range(3):
            b = rb.sample(256, ns, gamma)
            bo, bn = b.obs.cpu().numpy(), b.next_obs.cpu().numpy()
            for j in range(256):
                e, p, m = int(b.env[j]), int(b.pos[j]), int(b.steps[j])
                o, act, R, k, last, term = _brute(gt, e, p, ns, gamma)
                ok = (np.array_equal(bo[j], o) and int(b.action[j]) == act and k == m and np.array_equal(bn[j], last)
                      and bool(b.terminal[j]) == term and abs(float(b.reward[j]) - R) < 1e-4
                      and abs(float(b.discount[j]) - (0 if term else gamma ** k)) < 1e-5)
                bad += not ok
                checked += 1
    assert bad == 0, f"{bad}/{checked} sampled transitions differ"


def test_replay_rejects_stacks_deeper_than_the_ring():
    """k > capacity would make a stack reach past the oldest ring slot (the gather's slot arithmetic assumes
    k <= C): the C ABI refuses it before touching the device, and so does FrameReplay."""
    import ctypes

    from fast_mario_env_amd import _native
    L = ctypes.CDLL(_native.lib_path())
    L.mh_last_error.restype = ctypes.c_char_p
    P, I = ctypes.c_void_p, ctypes.c_int
    fake = P(1 << 20)                        # never dereferenced: validation fails first
    C, k, fb = 2, 4, 16
    rc = L.mh_replay_add(*[fake] * 7, I(1), I(C), I(fb), I(k), *[fake] * 6, P(0))
    assert rc == -1 and b"exceeds the ring capacity" in L.mh_last_error()
    rc = L.mh_replay_gather(*[fake] * 5, I(1), I(C), I(fb), I(k), fake, fake, I(1), I(1), *[fake] * 9, P(0))
    assert rc == -1 and b"exceeds the ring capacity" in L.mh_last_error()
    from fast_mario_env_amd.replay import FrameReplay
    with pytest.raises(ValueError, match="exceeds capacity"):
        FrameReplay(2, 1, k=4, device="cuda")
