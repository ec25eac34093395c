"""The FastVecEnv surface on the GPU (the reference's tests/test_api.py:54-98, ported): shapes and dtypes, the
zero-padded reset stack, list-of-dict infos with episode / final_obs / TimeLimit.truncated at the time
limit, env_offset equivalence, determinism, the monitor CSV rows, and set_buffers in both of its forms.
The CPU oracle is the checker for every value."""
import csv
import os

import numpy as np
import pytest
import torch

from build_roms import rom_path
from cpu_libs import OracleVec

pytestmark = pytest.mark.gpu

MINI = open(rom_path("vanilla"), "rb").read()


def _levels(names):
    from fast_mario_env_amd import decode_level
    return [decode_level(x) for x in names]


def test_shapes_infos_and_time_limit(tmp_path):
    """test_api.py:54-71: (3, 4, 84, 84) uint8 obs, zero-padded reset stack, float32 / bool outputs, the info
    keys, and at max_steps=20 every env truncated with episode l == 20, final_obs (4, 84, 84) and
    TimeLimit.truncated; here also every value against the oracle and the monitor CSV rows."""
    import fast_mario_env_amd as fme
    mon = tmp_path / "run"
    v = fme.FastVecEnv("1-1", 3, seed=0, max_steps=20, n_threads=2, rom=MINI, monitor_path=str(mon))
    ref = OracleVec(MINI, _levels(["1-1"] * 3), 3, seed=0, max_steps=20)
    obs = v.reset()
    assert obs.shape == (3, 4, 84, 84) and obs.dtype == np.uint8
    assert (obs[:, :3] == 0).all() and obs[:, 3].any()
    assert np.array_equal(obs, ref.reset())
    ended, episodes = 0, []
    for t in range(25):
        obs, r, te, tr, infos = v.step(np.full(3, 1))
        o1, r1, te1, tr1, i1 = ref.step(np.full(3, 1))
        assert r.dtype == np.float32 and te.dtype == bool and tr.dtype == bool and len(infos) == 3
        assert np.array_equal(obs, o1) and np.array_equal(r, r1) and np.array_equal(te, te1) and np.array_equal(tr, tr1)
        for i in range(3):
            assert set(fme.INFO_KEYS) <= set(infos[i])
            assert [infos[i][k] for k in fme.INFO_KEYS] == [int(x) for x in i1[i, :7]], (t, i)
            assert isinstance(infos[i]["flag_get"], bool)
        for i in np.flatnonzero(te | tr):
            ended += 1
            ep = infos[i]["episode"]
            assert infos[i]["final_obs"].shape == (4, 84, 84)
            assert np.array_equal(infos[i]["final_obs"], ref.fin[i])
            assert ep["l"] == 20 and infos[i]["TimeLimit.truncated"]
            assert ep["r"] == round(float(ref.ep_ret[i]), 6)
            assert ep["x_pos"] == infos[i]["x_pos"] and ep["flag_get"] == infos[i]["flag_get"]
            episodes.append(ep)
        for i in np.flatnonzero(~(te | tr)):
            assert "episode" not in infos[i] and "final_obs" not in infos[i]
    assert ended == 3
    assert v.bad_ops() == 0 and v.frames == ref.frames() > 0
    v.close()
    path = fme.MonitorCSV.resolve(str(mon))
    lines = open(path).read().splitlines()
    assert lines[0].startswith("#{") and '"t_start"' in lines[0]
    rows = list(csv.DictReader(lines[1:]))
    assert len(rows) == len(episodes) == 3
    for row, ep in zip(rows, episodes):
        assert float(row["r"]) == ep["r"] and int(row["l"]) == ep["l"] and int(row["x_pos"]) == ep["x_pos"]
        assert row["flag_get"] == str(ep["flag_get"]) and float(row["t"]) >= 0


def test_env_offset_matches_single_env():
    """test_api.py:89-98: envs 2..3 of a 4-env instance equal a 2-env instance with env_offset=2."""
    import fast_mario_env_amd as fme
    acts = np.random.default_rng(1).integers(0, 7, (40, 4))
    a = fme.FastVecEnv("1-1", 4, seed=2, sticky=0.25, noop_max=10, rom=MINI)
    b = fme.FastVecEnv("1-1", 2, seed=2, sticky=0.25, noop_max=10, env_offset=2, rom=MINI)
    oa, ob = a.reset(), b.reset()
    assert np.array_equal(oa[2:], ob)
    for x in acts:
        ra, rb = a.step(x), b.step(x[2:])
        assert np.array_equal(ra[0][2:], rb[0]) and np.array_equal(ra[1][2:], rb[1])
    a.close(); b.close()


def test_determinism():
    """test_api.py:74-86: the same seed gives the same trajectory (n_threads sizes the reference's pool and
    changes nothing here either)."""
    import fast_mario_env_amd as fme
    acts = np.random.default_rng(0).integers(0, 7, (60, 4))
    outs = []
    for threads in (0, 3):
        v = fme.FastVecEnv(["1-1", "1-2", "4-1", "8-4"], 4, seed=5, sticky=0.25, noop_max=10, n_threads=threads,
                           rom=MINI)
        o = [v.reset()]
        for x in acts:
            o.append(v.step(x)[0])
        outs.append(np.stack(o))
        v.close()
    assert np.array_equal(outs[0], outs[1])


def test_set_buffers_numpy_like_the_reference():
    """set_buffers with numpy arrays and the reference's int64 info / ep_len: reset and step write into them."""
    import fast_mario_env_amd as fme
    n, kw = 4, dict(seed=3, sticky=0.25, noop_max=5, max_steps=12)
    v = fme.FastVecEnv(["1-1", "4-1", "1-2", "8-4"], n, rom=MINI, **kw)
    ref = OracleVec(MINI, _levels(["1-1", "4-1", "1-2", "8-4"]), n, **kw)
    bufs = (np.zeros((n, 4, 84, 84), np.uint8), np.zeros((n, 4, 84, 84), np.uint8), np.zeros(n, np.float32),
            np.zeros(n, np.uint8), np.zeros(n, np.uint8), np.zeros((n, 10), np.int64), np.zeros(n, np.float64),
            np.zeros(n, np.int64))
    v.set_buffers(*bufs)
    v.reset()
    assert np.array_equal(bufs[0], ref.reset())
    rng = np.random.default_rng(2)
    ends = 0
    for _ in range(30):
        a = rng.integers(0, 7, n)
        v.step(a)
        ref.step(a)
        for mine, theirs in zip(bufs, (ref.obs, ref.fin, ref.rew, ref.term, ref.trunc, ref.info, ref.ep_ret, ref.ep_len)):
            assert np.array_equal(mine, theirs)
        ends += int((ref.term | ref.trunc).sum())
    assert ends > 0
    with pytest.raises(ValueError, match="info"):
        v.set_buffers(*bufs[:5], np.zeros((n, 10), np.float32), *bufs[6:])
    v.close()


def test_set_buffers_device_and_refusals():
    """Device buffers are written in place by the kernels; pageable host memory and misaligned buffers are
    refused with a message instead of being written by the GPU."""
    import fast_mario_env_amd as fme
    n = 2
    v = fme.FastVecEnv("1-1", n, seed=1, rom=MINI)
    z = lambda *s, dt: torch.zeros(*s, dtype=dt, device="cuda")  # noqa: E731
    dev = [z(n, 4, 84, 84, dt=torch.uint8), z(n, 4, 84, 84, dt=torch.uint8), z(n, dt=torch.float32),
           z(n, dt=torch.uint8), z(n, dt=torch.uint8), z(n, 10, dt=torch.int32), z(n, dt=torch.float64),
           z(n, dt=torch.int32)]
    v.set_buffers(*dev)
    v.reset()
    torch.cuda.synchronize()
    assert dev[0][:, 3].any() and not dev[0][:, :3].any()
    v.step(np.array([1, 2]))
    torch.cuda.synchronize()
    ref = OracleVec(MINI, _levels(["1-1"] * n), n, seed=1)
    ref.reset()
    ref.step(np.array([1, 2]))
    assert np.array_equal(dev[0].cpu().numpy(), ref.obs) and np.array_equal(dev[5].cpu().numpy(), ref.info)
    host = np.zeros((n, 4, 84, 84), np.uint8)                       # pageable host memory as a raw address
    addrs = [host.ctypes.data] + [int(t.data_ptr()) for t in dev[1:]]
    with pytest.raises(RuntimeError, match="pageable"):
        v.set_buffers(*addrs)
    addrs = [int(dev[0].data_ptr()) + 1] + [int(t.data_ptr()) for t in dev[1:]]
    with pytest.raises(RuntimeError, match="aligned"):
        v.set_buffers(*addrs)
    # the refusals left no stale error behind: the env still steps
    v.set_buffers(*dev)
    v.step(np.array([0, 0]))
    torch.cuda.synchronize()
    v.close()


def test_stack_kernels_on_4_byte_aligned_buffers():
    """Observation and final-observation stacks that are 4-byte but not 16-byte aligned take the 4-byte frame-stack
    kernel (16-byte aligned ones take the 16-byte one): the same observations, final observations and resets as the
    oracle over 40 steps with episode ends (max_steps=9)."""
    import fast_mario_env_amd as fme
    n = 3
    v = fme.FastVecEnv("1-1", n, seed=2, rom=MINI, max_steps=9)
    z = lambda *s, dt: torch.zeros(*s, dtype=dt, device="cuda")  # noqa: E731
    big = z(2 * n * 4 * 84 * 84 + 64, dt=torch.uint8)
    obs = big[4:4 + n * 4 * 84 * 84].view(n, 4, 84, 84)             # 4 bytes past a 16-byte boundary
    fin = big[n * 4 * 84 * 84 + 8:2 * n * 4 * 84 * 84 + 8].view(n, 4, 84, 84)
    assert obs.data_ptr() % 16 == 4 and fin.data_ptr() % 16 == 8
    rest = [z(n, dt=torch.float32), z(n, dt=torch.uint8), z(n, dt=torch.uint8), z(n, 10, dt=torch.int32),
            z(n, dt=torch.float64), z(n, dt=torch.int32)]
    v.set_buffers(obs, fin, *rest)
    ref = OracleVec(MINI, _levels(["1-1"] * n), n, seed=2, max_steps=9)
    v.reset()
    ref.reset()
    torch.cuda.synchronize()
    assert np.array_equal(obs.cpu().numpy(), ref.obs)
    ends = 0
    for t in range(40):
        a = np.array([t % 7, (3 * t) % 7, (5 * t + 1) % 7])
        v.step(a)
        ref.step(a)
        torch.cuda.synchronize()
        assert np.array_equal(obs.cpu().numpy(), ref.obs), t
        d = np.flatnonzero(ref.term | ref.trunc)
        ends += len(d)
        for i in d:
            assert np.array_equal(fin[i].cpu().numpy(), ref.fin[i]), (t, i)
    assert ends >= 6
    v.close()


class _StackLikeSb3:
    """SB3's VecFrameStack rule for channels-last Box observations, restated for this test (SB3 is not installed):
    reset zero-fills the stack and puts the frame last; each step shifts the stack one frame towards the front,
    and for an env that is done builds its terminal_observation as the stack's newest k-1 frames followed by the
    final frame, zero-fills the stack, then puts the new frame last."""

    def __init__(self, k):
        self.k = k

    def reset(self, o):
        self.s = np.zeros(o.shape[:3] + (self.k,), np.uint8)
        self.s[..., -1:] = o
        return self.s.copy()

    def step(self, o, dones, infos):
        self.s = np.roll(self.s, -1, axis=-1)
        for i in np.flatnonzero(dones):
            t = infos[i].get("terminal_observation")
            if t is not None:
                infos[i]["terminal_observation"] = np.concatenate([self.s[i, ..., :-1], t], axis=-1)
            self.s[i] = 0
        self.s[..., -1:] = o
        return self.s.copy()


def _fake_sb3(monkeypatch):
    """Minimal gymnasium.spaces and SB3 VecEnv base modules, enough for sb3_vec_env to build its class."""
    import sys
    import types

    class VecEnv:
        def __init__(self, num_envs, observation_space, action_space):
            self.num_envs, self.observation_space, self.action_space = num_envs, observation_space, action_space

        def step(self, actions):
            self.step_async(actions)
            return self.step_wait()

    class Box:
        def __init__(self, low, high, shape, dtype):
            self.low, self.high, self.shape, self.dtype = low, high, tuple(shape), dtype

    class Discrete:
        def __init__(self, n):
            self.n = n

    mods = {"gymnasium": types.ModuleType("gymnasium"), "gymnasium.spaces": types.ModuleType("gymnasium.spaces")}
    mods["gymnasium.spaces"].Box, mods["gymnasium.spaces"].Discrete = Box, Discrete
    mods["gymnasium"].spaces = mods["gymnasium.spaces"]
    for name in ("stable_baselines3", "stable_baselines3.common", "stable_baselines3.common.vec_env",
                 "stable_baselines3.common.vec_env.base_vec_env"):
        mods[name] = types.ModuleType(name)
    mods["stable_baselines3.common.vec_env.base_vec_env"].VecEnv = VecEnv
    for name, m in mods.items():
        monkeypatch.setitem(sys.modules, name, m)


def test_sb3_adapter(monkeypatch):
    """test_api.py:101-116 of the reference: single frames stacked by SB3's VecFrameStack rule equal the env's own
    stacks (stack_in_cpp=True), observations, dones and terminal observations, over 30 steps with time-limit
    ends (max_steps=12); the stacked env is also checked against the oracle."""
    import fast_mario_env_amd as fme
    _fake_sb3(monkeypatch)
    kw = dict(seed=0, max_steps=12, rom=MINI)
    single = fme.sb3_vec_env("1-1", 2, **kw)
    fast = fme.sb3_vec_env("1-1", 2, stack_in_cpp=True, **kw)
    assert single.observation_space.shape == (84, 84, 1) and fast.observation_space.shape == (4, 84, 84)
    assert single.action_space.n == 7 and single.num_envs == 2
    assert single.get_attr("x") == [None, None] and single.env_is_wrapped(object, indices=1) == [False]
    ref = OracleVec(MINI, _levels(["1-1"] * 2), 2, seed=0, max_steps=12)
    stack = _StackLikeSb3(4)
    o1, o2 = stack.reset(single.reset()), fast.reset()
    assert o1.shape == (2, 84, 84, 4) and o2.shape == (2, 4, 84, 84)
    assert np.array_equal(o1.transpose(0, 3, 1, 2), o2) and np.array_equal(o2, ref.reset())
    ends = 0
    for t in range(30):
        a = np.array([t % 7, (t * 3) % 7])
        s1, _, d1, i1 = single.step(a)
        o2, r2, d2, i2 = fast.step(a)
        o1 = stack.step(s1, d1, i1)
        ref.step(a)
        assert np.array_equal(o1.transpose(0, 3, 1, 2), o2) and np.array_equal(d1, d2)
        assert np.array_equal(o2, ref.obs) and np.array_equal(r2, ref.rew)
        for i in np.flatnonzero(d2):
            ends += 1
            assert np.array_equal(i1[i]["terminal_observation"].transpose(2, 0, 1), i2[i]["terminal_observation"])
            assert np.array_equal(i2[i]["terminal_observation"], ref.fin[i])
            assert "episode" not in i2[i]
            assert i2[i]["TimeLimit.truncated"] == bool(ref.trunc[i] and not ref.term[i])
    assert ends >= 4
    single.close(); fast.close()
