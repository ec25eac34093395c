"""PPO rollout harness (config 5 of the build's workloads; the reference's ppo/train.py rollout and GAE,
train.py:140-150): GAE against its recurrence written out element by element, the frame-deduplicated
stack rebuild against explicit frame stacking, and on the GPU a rollout whose stored observations, rewards
(with the timeout bootstrap) and episode starts are checked against the CPU oracle stepping its actions."""
import numpy as np
import pytest
import torch

from fast_mario_env_amd.rollout import Rollout, gae, gae_reference


def test_gae_matches_recurrence():
    rng = np.random.default_rng(5)
    T, n = 9, 6
    rew = rng.normal(size=(T, n)).astype(np.float32)
    val = rng.normal(size=(T, n)).astype(np.float32)
    start = rng.random((T, n)) < 0.25
    nv = rng.normal(size=n).astype(np.float32)
    ns = rng.random(n) < 0.3
    a, r = gae(torch.from_numpy(rew), torch.from_numpy(val), torch.from_numpy(start), torch.from_numpy(nv),
               torch.from_numpy(ns), 0.99, 0.95)
    ea, er = gae_reference(rew, val, start, nv, ns, 0.99, 0.95)
    assert np.allclose(a.numpy(), ea, rtol=1e-5, atol=1e-5) and np.allclose(r.numpy(), er, rtol=1e-5, atol=1e-5)
    # closed forms: no episode starts and lam = 1 -> discounted return minus value; lam = 0 -> one-step TD error
    s0 = np.zeros((T, n), bool)
    a1, _ = gae(torch.from_numpy(rew), torch.from_numpy(val), torch.from_numpy(s0), torch.from_numpy(nv),
                torch.zeros(n, dtype=torch.bool), 0.9, 1.0)
    disc = np.zeros((T, n)); g = nv.astype(np.float64)
    for t in reversed(range(T)):
        g = rew[t] + 0.9 * g; disc[t] = g
    assert np.allclose(a1.numpy(), disc - val, rtol=1e-4, atol=1e-4)
    a0, _ = gae(torch.from_numpy(rew), torch.from_numpy(val), torch.from_numpy(s0), torch.from_numpy(nv),
                torch.zeros(n, dtype=torch.bool), 0.9, 0.0)
    nxt = np.concatenate([val[1:], nv[None]], 0)
    assert np.allclose(a0.numpy(), rew + 0.9 * nxt - val, rtol=1e-5, atol=1e-5)


class _Stacker:
    """Explicit frame stacking of k frames with resets to [0, ..., 0, frame]."""
    def __init__(self, n, k):
        self.s = np.zeros((n, k, 84, 84), np.uint8)

    def push(self, frame, reset):
        self.s[:, :-1] = np.where(reset[:, None, None, None], 0, self.s[:, 1:])
        self.s[:, -1] = frame
        return self.s.copy()


def test_stack_rebuild_from_newest_frames():
    rng = np.random.default_rng(7)
    n, k, T = 5, 4, 11
    st = _Stacker(n, k)
    # history before the rollout, then the rollout's steps
    for _ in range(3):
        st.push(rng.integers(0, 255, (n, 84, 84), np.uint8), rng.random(n) < 0.3)
    ro = Rollout.__new__(Rollout)
    ro.torch, ro.k, ro.T = torch, k, T
    ro.frames = torch.zeros(T, n, 84, 84, dtype=torch.uint8)
    ro.start = torch.zeros(T, n, dtype=torch.bool)
    stacks = []
    for t in range(T):
        f = rng.integers(0, 255, (n, 84, 84), np.uint8)
        reset = rng.random(n) < 0.3
        if t == 0:
            reset[:] = False
        s = st.push(f, reset)
        if t == 0:
            ro.first = torch.from_numpy(s.copy())
        ro.frames[t] = torch.from_numpy(f)
        ro.start[t] = torch.from_numpy(reset)
        stacks.append(s)
    for t in range(T):
        assert np.array_equal(ro.obs(t).numpy(), stacks[t]), t


@pytest.mark.gpu
def test_rollout_vs_oracle():
    """A rollout's stored observations, actions, rewards and episode starts against the CPU oracle stepping the
    rollout's own actions; the time limit truncates episodes inside the rollout, and the stored reward of a
    truncated-not-terminated step is the oracle's reward plus gamma * V(oracle final_obs) (the reference
    trainer's timeout bootstrap, ppo/train.py:414-431). GAE over the stored arrays is checked against its
    recurrence."""
    from build_roms import rom_path
    from cpu_libs import OracleVec
    from fast_mario_env_amd import HipVecEnv, decode_level
    from fast_mario_env_amd.rollout import make_net
    rom = open(rom_path("vanilla"), "rb").read()
    names = ["1-1", "4-1", "8-4", "1-2", "2-3"] * 8
    kw = dict(seed=0, sticky=0.25, noop_max=30, max_steps=16, skip=4, frame_stack=4, maxpool=True)
    n, T, gamma = len(names), 24, 0.99
    env = HipVecEnv(names, n, rom=rom, **kw)
    env.reset()
    net = make_net(seed=0)
    ro = Rollout(env, net, T=T, seed=3, gamma=gamma)
    ro.collect()
    cpu = OracleVec(rom, [decode_level(x) for x in names], n, **kw)
    cpu.reset()
    n_boot, big_boot = 0, False
    for t in range(T):
        assert np.array_equal(ro.obs(t).cpu().numpy(), cpu.obs), t
        _, rew, term, trunc, _ = cpu.step(ro.act[t].cpu().numpy())
        want = torch.from_numpy(rew.copy()).cuda()
        boot = np.flatnonzero(trunc & ~term)
        if boot.size:
            n_boot += boot.size
            with torch.no_grad():
                _, v = net(torch.from_numpy(cpu.fin[boot].copy()).cuda())
            want[torch.from_numpy(boot).cuda()] += gamma * v
            big_boot |= bool((gamma * v).abs().max() > 0.01)
        # rewards are integers; the bootstrap term's bf16 trunk may take another convolution algorithm here
        assert torch.allclose(ro.rew[t], want, rtol=0, atol=2e-3), t
        nxt = ro.start[t + 1] if t + 1 < T else ro.next_start
        assert np.array_equal(nxt.cpu().numpy(), term | trunc), t
    assert n_boot > 0, "the time limit should truncate some episodes inside the rollout"
    assert big_boot, "the bootstrap terms should be large enough for the tolerance to tell them apart"
    assert ro.start[1:].any()
    adv, ret = ro.advantages()
    ea, er = gae_reference(*(x.cpu().numpy() for x in (ro.rew, ro.val, ro.start, ro.next_val, ro.next_start)),
                           gamma=gamma)
    assert np.allclose(adv.cpu().numpy(), ea, rtol=1e-4, atol=1e-4)
    assert np.allclose(ret.cpu().numpy(), er, rtol=1e-4, atol=1e-4)
    # the stored log-probs are the policy's on the rebuilt observations (same batch, same weights)
    lp_all = torch.log_softmax(net(ro.obs(T - 1))[0], -1)
    assert torch.allclose(lp_all.gather(-1, ro.act[T - 1][:, None]).squeeze(-1), ro.logp[T - 1], atol=1e-3)
    env.close()


@pytest.mark.gpu
def test_rollout_2048_envs_full_length_vs_oracle():
    """A full-length rollout (T = 128, the reference trainer's n_steps) of 2,048 envs over the 32 levels with the
    headline wrappers and a 100-step time limit (episodes end by death and by truncation inside the rollout, and
    the k_step waves beyond the first 64 compute their observations in-kernel): every env's stored observation
    stack, action-stepped reward (with the timeout bootstrap) and episode start against 16 oracle instances of
    128 envs on their own PCG64 streams (env_offset), stepping the rollout's recorded actions on a thread pool."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    from build_roms import rom_path
    from cpu_libs import OracleVec
    from fast_mario_env_amd import ALL_LEVELS, HipVecEnv, decode_level
    from fast_mario_env_amd.rollout import make_net
    rom = open(rom_path("vanilla"), "rb").read()
    names = [ALL_LEVELS[i % 32] for i in range(2048)]
    kw = dict(sticky=0.25, noop_max=30, max_steps=100, skip=4, frame_stack=4, maxpool=True)
    n, T, gamma, m = len(names), 128, 0.99, 128
    env = HipVecEnv(names, n, rom=rom, seed=0, **kw)
    env.reset()
    net = make_net(seed=0)
    ro = Rollout(env, net, T=T, seed=4, gamma=gamma)
    ro.collect()
    pool = ThreadPoolExecutor(min(16, os.cpu_count() or 1))
    cpu = list(pool.map(lambda k: OracleVec(rom, [decode_level(x) for x in names[k:k + m]], m, seed=0, env_offset=k,
                                            **kw), range(0, n, m)))
    list(pool.map(lambda c: c.reset(), cpu))
    acts = ro.act.cpu().numpy()
    n_boot = n_term = 0
    for t in range(T):
        o = np.concatenate([c.obs for c in cpu])
        bad = np.flatnonzero((ro.obs(t).cpu().numpy() != o).reshape(n, -1).any(1))
        assert bad.size == 0, (t, "obs of envs", bad[:8].tolist())
        outs = list(pool.map(lambda kc: [x.copy() for x in kc[1].step(acts[t, kc[0]:kc[0] + m])[1:4]] + [kc[1].fin.copy()],
                             zip(range(0, n, m), cpu)))
        rew, term, trunc, fin = (np.concatenate(z) for z in zip(*outs))
        want = torch.from_numpy(rew).cuda()
        boot = np.flatnonzero(trunc & ~term)
        if boot.size:
            n_boot += boot.size
            with torch.no_grad():
                _, v = net(torch.from_numpy(fin[boot]).cuda())
            want[torch.from_numpy(boot).cuda()] += gamma * v
        n_term += int(term.sum())
        # rewards are integers; the bootstrap term's bf16 trunk may take another convolution algorithm here
        assert torch.allclose(ro.rew[t], want, rtol=0, atol=2e-3), t
        nxt = ro.start[t + 1] if t + 1 < T else ro.next_start
        assert np.array_equal(nxt.cpu().numpy(), term | trunc), t
    pool.shutdown()
    assert n_boot > 0 and n_term > 0, (n_boot, n_term)
    assert env.bad_ops() == 0
    env.close()


@pytest.mark.gpu
@pytest.mark.parametrize("k,n", [(4, 97), (1, 5), (2, 3), (8, 2)])
def test_policy_input_kernel_matches_torch_scaling(k, n):
    # mh_policy_input against torch's own float32 scaling cast to bf16 (round to nearest even), bit for bit,
    # into a channels-last buffer; every byte value occurs
    from fast_mario_env_amd.rollout import policy_input
    g = torch.Generator(device="cuda").manual_seed(k)
    obs = torch.randint(0, 256, (n, k, 84, 84), dtype=torch.uint8, device="cuda", generator=g)
    obs.view(-1)[:256] = torch.arange(256, dtype=torch.uint8, device="cuda")
    out = torch.full((n, k, 84, 84), float("nan"), dtype=torch.bfloat16, device="cuda").to(memory_format=torch.channels_last)
    policy_input(obs, out)
    ref = (obs.float() * (1.0 / 255.0)).to(torch.bfloat16)
    assert torch.equal(out.view(torch.int16), ref.contiguous(memory_format=torch.channels_last).view(torch.int16))
    assert torch.equal(out.contiguous().view(torch.int16), ref.view(torch.int16))
    with pytest.raises(ValueError):
        policy_input(obs, out.contiguous() if k > 1 else out.float())   # NCHW (or float) output refused
    # a pageable host buffer is refused by the library before any kernel could touch it
    from fast_mario_env_amd._native import lib
    host = np.zeros(obs.numel() * 2, np.uint8)
    assert lib().mh_policy_input(obs.data_ptr(), host.ctypes.data, n, k, 0) == -1
    assert lib().mh_policy_input(host.ctypes.data, out.data_ptr(), n, k, 0) == -1


@pytest.mark.gpu
@pytest.mark.parametrize("n", [96, 4096])
def test_policy_forward_as_accurate_as_plain_bf16(n):
    # the GPU forward (the fused first layer, then channels-last bf16 convolutions) against the float32 network:
    # its error must be of the size of plain PyTorch's own bf16 forward (float32 scaling, NCHW, autocast), the two
    # bf16 pipelines rounding at different points; with autograd on it takes torch layers throughout. At 4,096
    # samples every convolution kernel's waves walk several tiles each (their launches are capped at 8 blocks
    # per CU), the shape of the rollout workload
    import torch.nn.functional as F

    from fast_mario_env_amd.rollout import make_net
    net = make_net(seed=1)
    obs = torch.randint(0, 256, (n, 4, 84, 84), dtype=torch.uint8, device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(5))

    def plain(bf16):
        x = obs.float().mul_(1.0 / 255.0)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=bf16):
            for c in net.convs:
                x = F.relu(F.conv2d(x, c.weight.contiguous(), c.bias, c.stride))
            h = F.relu(net.fc(x.flatten(1)))
        h = h.float()
        return net.pi(h), net.vf(h).squeeze(-1)

    with torch.no_grad():
        logits, value = net(obs)
        logits2, value2 = net(obs[:64])          # a second batch shape gets its own buffers
        ref_logits, ref_value = plain(False)
        bf_logits, bf_value = plain(True)
    for got, ref, bf in ((logits, ref_logits, bf_logits), (value, ref_value, bf_value)):
        err, bf_err = (got - ref).abs().max().item(), (bf - ref).abs().max().item()
        assert err <= 2.0 * bf_err + 1e-3, (err, bf_err)
        assert torch.allclose(got, ref, rtol=5e-2, atol=1e-2)
    # (the library's layers may pick other kernels, with other summation orders, for another batch size)
    assert torch.allclose(logits[:64], logits2, rtol=2e-2, atol=2e-3)
    with torch.no_grad():
        logits4, _ = net(obs[::2])               # a view that is not contiguous: the scaling kernel + torch layers
    assert torch.allclose(logits[::2], logits4, rtol=2e-2, atol=2e-3)
    logits3, value3 = net(obs)
    assert logits3.requires_grad
    for got, ref, bf in ((logits3.detach(), ref_logits, bf_logits), (value3.detach(), ref_value, bf_value)):
        assert (got - ref).abs().max().item() <= 2.0 * (bf - ref).abs().max().item() + 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 3, 50, 4096])
def test_policy_conv1_kernel_matches_torch(n):
    # the fused MFMA first layer against torch's: bf16 input (mh_policy_input), bf16 convolution with its bias
    # under autocast, ReLU. Both accumulate in float32 in different orders and torch rounds the convolution to
    # bf16 before adding the bias, so they agree to a bf16 rounding or two. At 4,096 samples (1.6M output pixels,
    # 51,200 tiles of 32) each wave of the persistent kernel walks several tiles, with the next tile's prefetch
    import torch.nn.functional as F

    from fast_mario_env_amd.rollout import make_net, policy_conv1, policy_input
    net = make_net(seed=2)
    g = torch.Generator(device="cuda").manual_seed(n)
    obs = torch.randint(0, 256, (n, 4, 84, 84), dtype=torch.uint8, device="cuda", generator=g)
    c = net.convs[0]
    with torch.no_grad():
        y = policy_conv1(obs, c.weight, c.bias)
        x = torch.empty(n, 4, 84, 84, dtype=torch.bfloat16, device="cuda").to(memory_format=torch.channels_last)
        policy_input(obs, x)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            ref = F.relu(F.conv2d(x, c.weight, c.bias, stride=4))
    assert y.shape == ref.shape and y.dtype == torch.bfloat16
    assert y.is_contiguous(memory_format=torch.channels_last)
    yf, rf = y.float(), ref.float()
    assert torch.allclose(yf, rf, rtol=1.6e-2, atol=2e-3), (yf - rf).abs().max().item()
    assert ((yf - rf).abs() <= 1.6e-2 * rf.abs() + 2e-3).float().mean() == 1.0
    assert (yf > 0).float().mean() > 0.2          # the layer is not trivially zero
    with pytest.raises(ValueError):
        policy_conv1(obs[:, :3].contiguous(), c.weight, c.bias)


@pytest.mark.gpu
@pytest.mark.parametrize("layer,n", [(2, 1), (2, 37), (2, 4096), (3, 1), (3, 37), (3, 4096)])
def test_policy_conv_kernels_match_torch(layer, n):
    # the fused MFMA second and third layers against torch's bf16 convolutions with bias under autocast and ReLU;
    # at 4,096 samples each wave of the persistent kernels walks several tiles, with the next tile's prefetch
    import torch.nn.functional as F

    from fast_mario_env_amd.rollout import make_net, policy_conv
    net = make_net(seed=4)
    c = net.convs[layer - 1]
    ci, hi = (32, 20) if layer == 2 else (64, 9)
    g = torch.Generator(device="cuda").manual_seed(layer * 100 + n)
    x = torch.rand(n, ci, hi, hi, generator=g, device="cuda").to(torch.bfloat16).to(memory_format=torch.channels_last)
    with torch.no_grad():
        y = policy_conv(x, c.weight, c.bias, layer)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            ref = F.relu(F.conv2d(x, c.weight, c.bias, stride=c.stride))
    assert y.shape == ref.shape and y.is_contiguous(memory_format=torch.channels_last)
    yf, rf = y.float(), ref.float()
    assert torch.allclose(yf, rf, rtol=1.6e-2, atol=4e-3), (yf - rf).abs().max().item()
    assert (yf > 0).float().mean() > 0.2
    with pytest.raises(ValueError):
        policy_conv(x.contiguous() if ci > 1 else x, c.weight, c.bias, layer)   # NCHW input refused
