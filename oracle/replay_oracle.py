"""CPU oracle for the frame-deduplicating replay ring -- TEST INFRASTRUCTURE ONLY.

A plain numpy restatement of the storage update and the batch assembly of the reference's FrameReplay
(src/fast_mario_env/replay.py), element by element, used by tests/ to check the HIP kernels
(mh_replay_add, mh_replay_gather) bit for bit. Nothing in the product imports it.

Parity pinning: tests/test_replay.py feeds it synthetic frame-stacked episodes (resets, terminations,
time-limit truncations, ring wrap-around) and checks every sampleable slot against the transitions as they
were added: the rebuilt obs / next_obs stacks, the action, the number of steps m, the terminal flag, and
the n-step return and discount against a float64 brute-force sum.
"""
from __future__ import annotations

import numpy as np


class ReplayOracle:
    """Ring of C single frames per env with age / action / reward / flags per slot (replay.py:43-60)."""

    def __init__(self, capacity_per_env: int, n_envs: int, k: int = 4, hw=(84, 84)):
        self.C, self.E, self.k, self.hw = int(capacity_per_env), int(n_envs), int(k), tuple(hw)
        self.frames = np.zeros((self.E, self.C, *self.hw), np.uint8)
        self.age = np.zeros((self.E, self.C), np.uint8)
        self.act = np.zeros((self.E, self.C), np.int16)
        self.rew = np.zeros((self.E, self.C), np.float32)
        self.flags = np.zeros((self.E, self.C), np.uint8)
        self.ptr = np.zeros(self.E, np.int64)
        self.new_ep = np.ones(self.E, bool)

    def _put(self, e: int, frame, age: int):
        """replay.py:68-74: the frame goes to slot ptr mod C with its age and cleared flags."""
        s = int(self.ptr[e]) % self.C
        self.frames[e, s] = frame
        self.age[e, s] = age
        self.flags[e, s] = 0
        self.ptr[e] += 1

    def add(self, obs, next_obs, action, reward, done, truncated=None):
        """replay.py:76-95, one env at a time."""
        obs, next_obs = np.asarray(obs, np.uint8), np.asarray(next_obs, np.uint8)
        done = np.asarray(done, bool).reshape(-1)
        trunc = np.zeros_like(done) if truncated is None else np.asarray(truncated, bool).reshape(-1)
        action = np.asarray(action).reshape(-1)
        reward = np.asarray(reward, np.float32).reshape(-1)
        for e in range(self.E):
            if self.new_ep[e]:
                self._put(e, obs[e, -1], 0)             # the stack of a new episode is zeros + this frame
            s = int(self.ptr[e] - 1) % self.C            # the slot the transition starts from
            self.act[e, s] = np.int16(np.int64(action[e]).astype(np.int16))
            self.rew[e, s] = reward[e]
            self.flags[e, s] = 1 | (2 if done[e] else 0) | (4 if done[e] and not trunc[e] else 0)
            self._put(e, next_obs[e, -1], min(int(self.age[e, s]) + 1, 255))
        self.new_ep = done.copy()

    def stack(self, e: int, q: int) -> np.ndarray:
        """replay.py:99-106: the k slots ending at q, zero where the slot precedes the episode start."""
        out = np.zeros((self.k, *self.hw), np.uint8)
        newest_age = int(self.age[e, q % self.C])
        for j in range(self.k):
            off = self.k - 1 - j
            if off <= newest_age:
                out[j] = self.frames[e, (q - off) % self.C]
        return out

    def n_step(self, e: int, p: int, n_step: int, gamma: float):
        """replay.py:131-142 in float32 with the reference's operation order."""
        R, alive, term, m = np.float32(0), np.float32(1), np.float32(0), 0
        for i in range(n_step):
            s = (p + i) % self.C
            f = int(self.flags[e, s])
            R = np.float32(R + np.float32(np.float32(alive * np.float32(gamma ** i)) * self.rew[e, s]))
            m += int(alive)
            term = max(term, np.float32(alive * np.float32(1.0 if f & 4 else 0.0)))
            alive = np.float32(alive * np.float32(0.0 if f & 2 else 1.0))
        disc = np.float32(np.float32(gamma ** m) * np.float32(1 - term))
        return R, m, term, disc

    def assemble(self, env, pos, n_step: int = 1, gamma: float = 0.99) -> dict:
        """The batch of (env, pos) pairs (replay.py:143-145)."""
        env, pos = np.asarray(env, np.int64), np.asarray(pos, np.int64)
        B = len(env)
        out = {"obs": np.zeros((B, self.k, *self.hw), np.uint8), "next_obs": np.zeros((B, self.k, *self.hw), np.uint8),
               "action": np.zeros(B, np.int64), "reward": np.zeros(B, np.float32), "discount": np.zeros(B, np.float32),
               "terminal": np.zeros(B, np.float32), "steps": np.zeros(B, np.int64)}
        for b in range(B):
            e, p = int(env[b]), int(pos[b])
            R, m, term, disc = self.n_step(e, p, n_step, gamma)
            out["obs"][b] = self.stack(e, p)
            out["next_obs"][b] = self.stack(e, p + m)
            out["action"][b] = int(self.act[e, p % self.C])
            out["reward"][b], out["steps"][b], out["terminal"][b], out["discount"][b] = R, m, term, disc
        return out

    def sampleable(self, n_step: int):
        """Every (env, pos) the reference's sampler can return: pos in [max(ptr - C + k - 1, 0),
        ptr - 1 - n_step] with flag bit 1 set (replay.py:112-127)."""
        pairs = []
        for e in range(self.E):
            lo, hi = max(int(self.ptr[e]) - self.C + self.k - 1, 0), int(self.ptr[e]) - 1 - n_step
            pairs += [(e, p) for p in range(lo, hi + 1) if self.flags[e, p % self.C] & 1]
        return pairs
