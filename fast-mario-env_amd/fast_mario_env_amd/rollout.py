"""PPO rollout harness on the GPU env: the device path of the reference's CudaMarioBackend and the rollout
half of its trainer (src/fast_mario_env/ppo/backends.py:127-162, ppo/train.py:120-150 and 398-441).

- `NatureAC`: the Nature-CNN actor-critic of the reference's ppo/model.py:13-38 (conv 32@8x8/4, 64@4x4/2,
  64@3x3/1, fc 512, a 7-way policy head and a value head; orthogonal init, gains sqrt(2) / 0.01 / 1). The
  trunk runs under bf16 autocast with channels-last convolutions on the GPU, the two heads in fp32.
- `Rollout`: T steps of N envs. The policy reads the env's observation tensor in place (no copy), samples
  with the Gumbel-max trick from its own torch.Generator, and the actions go back to the env on the same
  stream; the only host synchronization in a step is the timeout-bootstrap check below.
- Frame-deduplicated storage: a step stores only its newest 84x84 frame and whether its stack starts a new
  episode (a reset observation is [0, 0, 0, frame]); `obs(t)` rebuilds the (N, 4, 84, 84) stack of step t.
  32,768 envs x 128 steps then take 29.6 GB instead of 118 GB.
- Timeout bootstrap (train.py:414-431, the device-backend branch): where an episode was truncated by the time
  limit and not terminated, the stored reward is r + gamma * V(final_obs), V evaluated on the final
  observation stacks of those envs. As in the reference, finding them costs one small host sync per step.
- `gae`: generalized advantage estimation over the stored rewards, values and episode starts, with the
  reference's convention (train.py:140-150): the bootstrap of step t is cut where step t + 1 starts an episode.

The env-kernel share of a rollout is timed with events on the stream both run on.
"""
from __future__ import annotations

import math

import numpy as np

N_ACTIONS = 7


def _torch():
    import torch
    return torch


def policy_input(obs_u8, out):
    """Scale uint8 (B, k, 84, 84) observation stacks into `out`, a bf16 (B, k, 84, 84) channels-last tensor on the
    same GPU: bf16(float(v) * float(1/255)), rounded to nearest even, by the library's HIP kernel."""
    torch = _torch()
    from ._native import check, lib
    if (obs_u8.dtype != torch.uint8 or out.dtype != torch.bfloat16 or tuple(obs_u8.shape) != tuple(out.shape)
            or obs_u8.dim() != 4 or tuple(obs_u8.shape[2:]) != (84, 84) or not obs_u8.is_contiguous()
            or not out.is_contiguous(memory_format=torch.channels_last) or obs_u8.device != out.device):
        raise ValueError("policy_input: needs a contiguous uint8 (B, k, 84, 84) tensor and a bf16 channels-last "
                         "tensor of the same shape on the same GPU")
    check(lib().mh_policy_input(obs_u8.data_ptr(), out.data_ptr(), obs_u8.shape[0], obs_u8.shape[1],
                                torch.cuda.current_stream(obs_u8.device).cuda_stream), "mh_policy_input")
    return out


def policy_conv1(obs_u8, weight, bias, out=None):
    """relu(conv2d(bf16(obs / 255), weight, bias, stride 4)) of the Nature CNN's first layer by the library's MFMA
    kernel: obs uint8 (B, 4, 84, 84) contiguous on a GPU, weight (32, 4, 8, 8) and bias (32) in any float dtype
    (taken as bf16, as autocast takes them); returns (or fills) a bf16 (B, 32, 20, 20) channels-last tensor."""
    torch = _torch()
    from ._native import check, lib
    if (obs_u8.dtype != torch.uint8 or obs_u8.dim() != 4 or tuple(obs_u8.shape[1:]) != (4, 84, 84)
            or not obs_u8.is_contiguous() or tuple(weight.shape) != (32, 4, 8, 8) or tuple(bias.shape) != (32,)):
        raise ValueError("policy_conv1: needs a contiguous uint8 (B, 4, 84, 84) tensor, a (32, 4, 8, 8) weight and a "
                         "(32,) bias")
    w = weight.detach().to(device=obs_u8.device, dtype=torch.bfloat16).contiguous()
    b = bias.detach().to(device=obs_u8.device, dtype=torch.bfloat16).contiguous()
    n = obs_u8.shape[0]
    if out is None:
        out = torch.empty(n, 32, 20, 20, dtype=torch.bfloat16, device=obs_u8.device).to(memory_format=torch.channels_last)
    if (out.dtype != torch.bfloat16 or tuple(out.shape) != (n, 32, 20, 20)
            or not out.is_contiguous(memory_format=torch.channels_last)):
        raise ValueError("policy_conv1: out must be a bf16 (B, 32, 20, 20) channels-last tensor")
    check(lib().mh_policy_conv1(obs_u8.data_ptr(), w.data_ptr(), b.data_ptr(), out.data_ptr(), n,
                                torch.cuda.current_stream(obs_u8.device).cuda_stream), "mh_policy_conv1")
    return out


_CONV_SHAPES = {2: ((64, 32, 4, 4), (32, 20, 20), (64, 9, 9)), 3: ((64, 64, 3, 3), (64, 9, 9), (64, 7, 7))}


def policy_conv(x, weight, bias, layer, out=None):
    """relu(conv2d(x, weight, bias)) of the Nature CNN's second (layer=2: 4x4 stride 2) or third (layer=3: 3x3
    stride 1) convolution by the library's MFMA kernel: x a bf16 channels-last (B, C, H, H) tensor on a GPU,
    weight (64, C, k, k) and bias (64) in any float dtype (taken as bf16, as autocast takes them); returns (or
    fills) the bf16 channels-last output."""
    torch = _torch()
    from ._native import check, lib
    wshape, ishape, oshape = _CONV_SHAPES[layer]
    n = x.shape[0]
    if (x.dtype != torch.bfloat16 or tuple(x.shape[1:]) != ishape or not x.is_contiguous(memory_format=torch.channels_last)
            or tuple(weight.shape) != wshape or tuple(bias.shape) != (64,)):
        raise ValueError(f"policy_conv layer {layer}: needs a bf16 channels-last (B, {ishape[0]}, {ishape[1]}, {ishape[2]}) "
                         f"input, a {wshape} weight and a (64,) bias")
    w = weight.detach().to(device=x.device, dtype=torch.bfloat16).permute(0, 2, 3, 1).contiguous()
    b = bias.detach().to(device=x.device, dtype=torch.bfloat16).contiguous()
    if out is None:
        out = torch.empty((n,) + oshape, dtype=torch.bfloat16, device=x.device).to(memory_format=torch.channels_last)
    if out.dtype != torch.bfloat16 or tuple(out.shape) != (n,) + oshape or not out.is_contiguous(memory_format=torch.channels_last):
        raise ValueError(f"policy_conv layer {layer}: out must be a bf16 channels-last (B,) + {oshape} tensor")
    check(lib().mh_policy_conv(x.data_ptr(), w.data_ptr(), b.data_ptr(), out.data_ptr(), n, layer,
                               torch.cuda.current_stream(x.device).cuda_stream), "mh_policy_conv")
    return out


def make_net(n_actions: int = N_ACTIONS, in_ch: int = 4, seed: int = 0, device="cuda"):
    """The Nature-CNN actor-critic with the reference's architecture and initialisation, random weights."""
    torch = _torch()
    nn = torch.nn
    F = torch.nn.functional

    class NatureAC(nn.Module):
        def __init__(self):
            super().__init__()
            self.convs = nn.ModuleList([nn.Conv2d(in_ch, 32, 8, 4), nn.Conv2d(32, 64, 4, 2), nn.Conv2d(64, 64, 3, 1)])
            self.fc = nn.Linear(64 * 7 * 7, 512)
            self.pi = nn.Linear(512, n_actions)
            self.vf = nn.Linear(512, 1)
            for m in list(self.convs) + [self.fc]:
                nn.init.orthogonal_(m.weight, math.sqrt(2.0))
                nn.init.zeros_(m.bias)
            nn.init.orthogonal_(self.pi.weight, 0.01)
            nn.init.zeros_(self.pi.bias)
            nn.init.orthogonal_(self.vf.weight, 1.0)
            nn.init.zeros_(self.vf.bias)
            self._inputs = {}

        def _input(self, shape, device):
            """The bf16 channels-last input buffer of a batch shape (reused by every call of that shape)."""
            key = (tuple(shape), str(device))
            buf = self._inputs.get(key)
            if buf is None:
                buf = torch.empty(shape, dtype=torch.bfloat16, device=device).to(memory_format=torch.channels_last)
                self._inputs[key] = buf
            return buf

        def forward(self, obs_u8):
            """uint8 (B, 4, 84, 84) -> logits f32 (B, A), value f32 (B,).

            On the GPU each convolution is one HIP kernel on the matrix cores with float32 accumulation, its bias
            and its ReLU (mh_policy_conv1, mh_policy_conv): the first one scales the observation to
            bf16(float(v) * float(1/255)) (the value autocast gives the float32 scaling of the CPU path); the
            activations are bf16 channels-last. Other stack depths take mh_policy_input's scaling
            into a bf16 channels-last buffer and the convolutions. Calls of one batch shape share the buffers.
            With autograd on, the scaled input takes a buffer of its own and every layer is a torch layer."""
            convs = list(self.convs)
            grad = torch.is_grad_enabled()   # the fused layer has no backward, and a shared buffer must not be
            if obs_u8.is_cuda and grad:      # overwritten while autograd holds it: the plain path, own buffers
                x = torch.empty(obs_u8.shape, dtype=torch.bfloat16, device=obs_u8.device).to(
                    memory_format=torch.channels_last)
                policy_input(obs_u8.contiguous(), x)
            elif obs_u8.is_cuda and obs_u8.shape[1] == 4 and obs_u8.is_contiguous():
                # the three convolutions with their input scaling, biases and ReLUs as MFMA kernels
                # (mh_policy_conv1, mh_policy_conv); the fully connected layer takes the last one's
                # channels-last output as it lies, with its weight's columns permuted to (h, w, c) order
                B, dev = obs_u8.shape[0], obs_u8.device
                x = policy_conv1(obs_u8, convs[0].weight, convs[0].bias, self._input((B, 32, 20, 20), dev))
                x = policy_conv(x, convs[1].weight, convs[1].bias, 2, self._input((B, 64, 9, 9), dev))
                x = policy_conv(x, convs[2].weight, convs[2].bias, 3, self._input((B, 64, 7, 7), dev))
                wfc = self.fc.weight.view(512, 64, 7, 7).permute(0, 2, 3, 1).reshape(512, 64 * 7 * 7)
                with torch.autocast("cuda", dtype=torch.bfloat16):
                    h = F.relu(F.linear(x.permute(0, 2, 3, 1).reshape(B, 64 * 7 * 7), wfc, self.fc.bias))
                h = h.float()
                return self.pi(h), self.vf(h).squeeze(-1)
            elif obs_u8.is_cuda:
                # other stack depths, and views that are not contiguous (policy_input takes contiguous stacks)
                x = self._input(obs_u8.shape, obs_u8.device)
                policy_input(obs_u8.contiguous(), x)
            else:
                x = obs_u8.float().mul_(1.0 / 255.0)
            with torch.autocast("cuda", dtype=torch.bfloat16, enabled=x.is_cuda):
                for c in convs:
                    x = F.relu(c(x))
                h = F.relu(self.fc(x.flatten(1)))
            h = h.float()
            return self.pi(h), self.vf(h).squeeze(-1)

        @torch.no_grad()
        def act(self, obs_u8, generator=None):
            """Action (Gumbel-max sample, i.e. a categorical draw), its log-probability and the value."""
            logits, v = self(obs_u8)
            logp = F.log_softmax(logits, -1)
            u = torch.rand(logits.shape, generator=generator, device=logits.device).clamp_(1e-20, 1.0)
            a = (logp - torch.log(-torch.log(u))).argmax(-1)
            return a, logp.gather(-1, a[:, None]).squeeze(-1), v

    torch.manual_seed(seed)
    net = NatureAC().to(device)
    if torch.device(device).type == "cuda":
        net = net.to(memory_format=torch.channels_last)   # NHWC convolutions (MIOpen's faster layout here)
    return net


def gae(rew, val, start, next_val, next_start, gamma: float = 0.99, lam: float = 0.95):
    """Advantages and returns (T, N) from rewards, values and episode starts (T, N) plus the bootstrap value and
    start flag of the step after the last: delta_t = r_t + gamma v_{t+1} (1 - s_{t+1}) - v_t,
    A_t = delta_t + gamma lam (1 - s_{t+1}) A_{t+1}."""
    torch = _torch()
    T = rew.shape[0]
    adv = torch.zeros_like(rew)
    last = torch.zeros_like(next_val)
    for t in reversed(range(T)):
        nv, ns = (next_val, next_start) if t == T - 1 else (val[t + 1], start[t + 1])
        keep = 1.0 - ns.float()
        delta = rew[t] + gamma * nv * keep - val[t]
        last = delta + (gamma * lam) * keep * last
        adv[t] = last
    return adv, adv + val


class Rollout:
    """T-step rollouts of `env` (a HipVecEnv) under `net`, stored frame-deduplicated on the env's device."""

    def __init__(self, env, net, T: int = 128, seed: int = 3, gamma: float = 0.99, bootstrap_timeouts: bool = True):
        torch = self.torch = _torch()
        self.env, self.net, self.T = env, net, T
        self.gamma, self.bootstrap_timeouts = gamma, bootstrap_timeouts
        n, dev = env.n, env.dev
        self.k = env.k
        self.gen = torch.Generator(device=dev)
        self.gen.manual_seed(seed)
        self.frames = torch.zeros(T, n, 84, 84, dtype=torch.uint8, device=dev)   # newest frame of each step
        self.start = torch.zeros(T, n, dtype=torch.bool, device=dev)              # the step's stack is a reset stack
        self.first = torch.zeros(n, self.k, 84, 84, dtype=torch.uint8, device=dev)  # full stack of step 0
        self.act = torch.zeros(T, n, dtype=torch.int64, device=dev)
        self.logp = torch.zeros(T, n, device=dev)
        self.val = torch.zeros(T, n, device=dev)
        self.rew = torch.zeros(T, n, device=dev)
        self.next_val = torch.zeros(n, device=dev)
        self.next_start = torch.zeros(n, dtype=torch.bool, device=dev)
        self._starting = torch.ones(n, dtype=torch.bool, device=dev)   # the current obs is a reset stack
        self.env_ms = 0.0

    def collect(self):
        """One rollout; the env continues from where the last one stopped. Returns the env-kernel time in ms
        (measured with events on the stream; reading it synchronizes)."""
        torch, env = self.torch, self.env
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(self.T)]
        self.first.copy_(env.obs)
        for t in range(self.T):
            obs = env.obs                                    # the env's buffer, read in place
            self.frames[t].copy_(obs[:, -1])
            self.start[t].copy_(self._starting)
            a, lp, v = self.net.act(obs, self.gen)
            self.act[t].copy_(a)
            self.logp[t].copy_(lp)
            self.val[t].copy_(v)
            ev[t][0].record()
            _, rew, term, trunc, _ = env.step(self.act[t])
            ev[t][1].record()
            self.rew[t].copy_(rew)
            if self.bootstrap_timeouts:
                self._bootstrap(t, term, trunc)
            torch.logical_or(term, trunc, out=self._starting)   # the next obs is a reset stack
        _, _, v = self.net.act(env.obs, self.gen)
        self.next_val.copy_(v)
        self.next_start.copy_(self._starting)
        torch.cuda.synchronize(env.dev)
        self.env_ms = sum(a.elapsed_time(b) for a, b in ev)
        return self.env_ms

    def _bootstrap(self, t: int, term, trunc):
        """rew[t] += gamma * V(final_obs) where the time limit cut an episode that did not terminate."""
        torch = self.torch
        tmask = trunc & ~term
        if not bool(tmask.any()):            # rare (time limit): one small host sync
            return
        ti = tmask.nonzero().squeeze(-1)
        with torch.no_grad():
            _, v = self.net(self.env.final_obs[ti])
        self.rew[t, ti] += self.gamma * v

    def obs(self, t: int):
        """The (N, k, 84, 84) observation stack of step t, rebuilt from the stored frames."""
        torch = self.torch
        out = torch.zeros_like(self.first)
        out[:, -1] = self.frames[t]
        alive = ~self.start[t]               # the stack still continues one step further back
        for j in range(1, self.k):
            if t - j >= 0:
                out[:, -1 - j] = torch.where(alive[:, None, None], self.frames[t - j], 0)
                alive = alive & ~self.start[t - j]
            else:                            # before the rollout: the stack of step 0
                out[:, -1 - j] = torch.where(alive[:, None, None], self.first[:, -1 - (j - t)], 0)
        return out

    def advantages(self, gamma: float | None = None, lam: float = 0.95):
        g = self.gamma if gamma is None else gamma
        return gae(self.rew, self.val, self.start, self.next_val, self.next_start, g, lam)


def gae_reference(rew, val, start, next_val, next_start, gamma=0.99, lam=0.95):
    """The recurrence element by element in numpy (float64), for checking `gae`."""
    T, n = rew.shape
    adv = np.zeros((T, n))
    for i in range(n):
        last = 0.0
        for t in reversed(range(T)):
            nv, ns = (next_val[i], next_start[i]) if t == T - 1 else (val[t + 1, i], start[t + 1, i])
            keep = 0.0 if ns else 1.0
            last = rew[t, i] + gamma * nv * keep - val[t, i] + gamma * lam * keep * last
            adv[t, i] = last
    return adv, adv + val
