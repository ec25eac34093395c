"""Frame-deduplicating replay buffer on the GPU, mirroring the reference's FrameReplay
(src/fast_mario_env/replay.py:43-145): same constructor, add/sample/size/nbytes and Batch fields.

Each env keeps a ring of C single frames plus per-slot age, action, reward and flags; a k-frame stack is
rebuilt at sample time from the k newest slots, with the slots before the episode start zeroed, which
reproduces the zero-padded reset stacks of the env. Terminal frames are stored as slots of their own,
so time-limit truncation bootstraps correctly.

The storage is device tensors owned here; the two hot operations are HIP kernels of libmario_hip.so:
- `mh_replay_add`: one workgroup per env writes the newest frame(s) of the obs / next_obs stacks into the
  ring and updates the slot metadata, the write pointer and the new-episode flag on the device (no host
  state, no synchronization);
- `mh_replay_gather`: one workgroup per output frame assembles a sampled batch (obs and next_obs stacks,
  n-step return, discount, terminal, steps, action) in a single launch.
The sampled (env, slot) pairs are drawn with the reference's sequence of torch generator calls
(replay.py:112-129: a uniform env among those with data, a uniform slot in its live window, rejection of
slots that do not start a transition), so a seeded buffer draws what the reference draws.
"""
from __future__ import annotations

from typing import NamedTuple

import numpy as np

from ._native import lib
from .env import _ptr, _stream, _torch


class Batch(NamedTuple):
    obs: object        # (B, k, H, W) uint8
    action: object     # (B,) int64
    reward: object     # (B,) float32, n-step discounted sum
    next_obs: object   # (B, k, H, W) uint8, the stack m <= n_step steps later
    discount: object   # (B,) float32 = gamma^m (1 - terminal)
    terminal: object   # (B,) float32, true termination (not truncation)
    steps: object      # (B,) int64 m
    env: object        # (B,) env index
    pos: object        # (B,) absolute slot index


def _check(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"{what}: {lib().mh_last_error().decode()}")


class FrameReplay:
    """Replay ring of `capacity_per_env` frames for each of `n_envs` envs, k-frame stacks of hw frames."""

    def __init__(self, capacity_per_env: int, n_envs: int, k: int = 4, hw=(84, 84), device="cuda", seed=None):
        self.C, self.E, self.k, self.hw = int(capacity_per_env), int(n_envs), int(k), tuple(hw)
        self.fb = self.hw[0] * self.hw[1]
        if self.C < 2 or self.E < 1 or self.k < 1 or self.fb % 16:
            raise ValueError("FrameReplay needs capacity_per_env >= 2, n_envs >= 1, k >= 1 and H*W a multiple of 16")
        if self.k > self.C:
            raise ValueError(f"FrameReplay: stack depth k={self.k} exceeds capacity_per_env={self.C} (a stack would "
                             "reach past the oldest frame the ring keeps)")
        torch = self.torch = _torch()
        self.dev = torch.device(device)
        if self.dev.type != "cuda":
            raise ValueError("FrameReplay keeps its ring in GPU memory: device must be a ROCm GPU")
        E, C, d = self.E, self.C, self.dev
        self.frames = torch.zeros((E, C, *self.hw), dtype=torch.uint8, device=d)
        self.age = torch.zeros((E, C), dtype=torch.uint8, device=d)
        self.act = torch.zeros((E, C), dtype=torch.int16, device=d)
        self.rew = torch.zeros((E, C), dtype=torch.float32, device=d)
        self.flags = torch.zeros((E, C), dtype=torch.uint8, device=d)   # 1 valid start, 2 done, 4 terminal
        self._ptr = torch.zeros(E, dtype=torch.int64, device=d)        # slots written per env
        self._new_ep = torch.ones(E, dtype=torch.uint8, device=d)
        self.g = torch.Generator(device=d)
        self.g.manual_seed(int(np.random.SeedSequence(seed).generate_state(1)[0]))
        self._err = torch.zeros(1, dtype=torch.int32, device=d)
        self._gpow = {}
        self.n_transitions = 0

    @property
    def ptr(self) -> np.ndarray:
        """Absolute number of slots written per env (a host copy; synchronizes)."""
        return self._ptr.cpu().numpy()

    @property
    def new_ep(self) -> np.ndarray:
        return self._new_ep.cpu().numpy().astype(bool)

    # ------------------------------------------------------------------ add
    def _dev(self, x, dtype=None):
        torch = self.torch
        if isinstance(x, torch.Tensor):
            return x.to(self.dev, dtype=dtype, non_blocking=True)
        return torch.as_tensor(np.ascontiguousarray(x), device=self.dev, dtype=dtype)

    def _stacks(self, x):
        t = self._dev(x, self.torch.uint8).contiguous()
        if tuple(t.shape) != (self.E, self.k, *self.hw):
            raise ValueError(f"expected ({self.E}, {self.k}, {self.hw[0]}, {self.hw[1]}) stacks, got {tuple(t.shape)}")
        return t

    def add(self, obs, next_obs, action, reward, done, truncated=None):
        """obs / next_obs: (N, k, H, W) stacks (next_obs is the terminal stack of a finished env);
        done = terminated | truncated; truncated marks time-limit ends (bootstrapped)."""
        torch = self.torch
        o, o2 = self._stacks(obs), self._stacks(next_obs)
        a = self._dev(action).reshape(-1).to(torch.int64).contiguous()
        r = self._dev(reward, torch.float32).reshape(-1).contiguous()
        dn = self._dev(done).reshape(-1).to(torch.uint8).contiguous()
        tr = torch.zeros_like(dn) if truncated is None else self._dev(truncated).reshape(-1).to(torch.uint8).contiguous()
        for name, t in (("action", a), ("reward", r), ("done", dn), ("truncated", tr)):
            if t.numel() != self.E:
                raise ValueError(f"{name} must have n_envs = {self.E} entries, got {t.numel()}")
        _check(lib().mh_replay_add(_ptr(self.frames), _ptr(self.age), _ptr(self.act), _ptr(self.rew),
                                   _ptr(self.flags), _ptr(self._ptr), _ptr(self._new_ep), self.E, self.C, self.fb,
                                   self.k, _ptr(o), _ptr(o2), _ptr(a), _ptr(r), _ptr(dn), _ptr(tr),
                                   _stream(torch, self.dev)), "mh_replay_add")
        self.n_transitions += self.E

    # --------------------------------------------------------------- sample
    def size(self) -> int:
        return int(min(self.n_transitions, self.E * self.C))

    def _gamma_pow(self, n_step: int, gamma: float):
        key = (n_step, float(gamma))
        t = self._gpow.get(key)
        if t is None:
            # float32(gamma ** i): the Python-float powers the reference multiplies its float32 tensors by
            t = self.torch.tensor([float(gamma) ** i for i in range(n_step + 1)], dtype=self.torch.float32, device=self.dev)
            self._gpow[key] = t
        return t

    def draw(self, batch: int, n_step: int = 1):
        """(env, pos) of `batch` transitions: env uniform among the envs with a sampleable window, pos uniform
        in [max(ptr - C + k - 1, 0), ptr - 1 - n_step], redrawn while the slot does not start a transition."""
        torch, C, d = self.torch, self.C, self.dev
        lo = torch.clamp(self._ptr - C + self.k - 1, min=0)      # the k-1 frames behind pos are still in the ring
        hi = self._ptr - 1 - n_step                               # the frame after pos + n_step - 1 is written
        cand = torch.nonzero(hi >= lo).flatten()
        if len(cand) == 0:
            raise ValueError("not enough data in buffer")
        env = torch.empty(batch, dtype=torch.long, device=d)
        pos = torch.empty(batch, dtype=torch.long, device=d)
        open_rows = torch.arange(batch, device=d)
        for _ in range(64):
            n = len(open_rows)
            ee = cand[torch.randint(len(cand), (n,), device=d, generator=self.g)]
            width = (hi[ee] - lo[ee] + 1).double()
            pp = lo[ee] + (torch.rand(n, device=d, generator=self.g, dtype=torch.float64) * width).long()
            ok = (self.flags[ee, pp % C] & 1).bool()
            env[open_rows[ok]] = ee[ok]
            pos[open_rows[ok]] = pp[ok]
            open_rows = open_rows[~ok]
            if len(open_rows) == 0:
                return env, pos
        raise RuntimeError("sampling failed")

    def gather(self, env, pos, n_step: int = 1, gamma: float = 0.99) -> Batch:
        """The batch of the transitions at (env, pos), assembled on the device in one kernel."""
        torch, d, B = self.torch, self.dev, int(env.numel())
        env = env.to(d, torch.int64).contiguous()
        pos = pos.to(d, torch.int64).contiguous()
        obs = torch.empty((B, self.k, *self.hw), dtype=torch.uint8, device=d)
        nxt = torch.empty_like(obs)
        action = torch.empty(B, dtype=torch.int64, device=d)
        reward = torch.empty(B, dtype=torch.float32, device=d)
        disc = torch.empty(B, dtype=torch.float32, device=d)
        term = torch.empty(B, dtype=torch.float32, device=d)
        steps = torch.empty(B, dtype=torch.int64, device=d)
        _check(lib().mh_replay_gather(_ptr(self.frames), _ptr(self.age), _ptr(self.act), _ptr(self.rew),
                                      _ptr(self.flags), self.E, self.C, self.fb, self.k, _ptr(env), _ptr(pos), B,
                                      int(n_step), _ptr(self._gamma_pow(int(n_step), gamma)), _ptr(obs), _ptr(nxt),
                                      _ptr(action), _ptr(reward), _ptr(disc), _ptr(term), _ptr(steps),
                                      _ptr(self._err), _stream(torch, d)), "mh_replay_gather")
        return Batch(obs, action, reward, nxt, disc, term, steps, env, pos)

    def sample(self, batch: int, n_step: int = 1, gamma: float = 0.99) -> Batch:
        env, pos = self.draw(batch, n_step)
        return self.gather(env, pos, n_step, gamma)

    def check_errors(self):
        """Raises if a gather was given an (env, pos) outside the ring (synchronizes)."""
        if int(self._err.item()):
            self._err.zero_()
            raise IndexError("FrameReplay.gather: an (env, pos) pair was outside the ring")

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.frames, self.age, self.act, self.rew, self.flags))
