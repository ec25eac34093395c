"""Stable-Baselines3 VecEnv over FastVecEnv: the reference's `sb3_vec_env` (src/fast_mario_env/sb3.py:10-71).

    from fast_mario_env_amd import sb3_vec_env
    from stable_baselines3.common.vec_env import VecFrameStack, VecMonitor
    venv = VecFrameStack(VecMonitor(sb3_vec_env("1-1", 8, seed=0)), 4)     # SB3 stacks single frames
    venv = sb3_vec_env("1-1", 8, seed=0, stack_in_cpp=True)                 # the GPU stacks them

Two observation layouts, as in the reference:
* single frames (default): (84, 84, 1) channels-last uint8, gym-super-mario-bros + WarpFrame's layout, for SB3's
  own VecFrameStack / VecMonitor;
* `stack_in_cpp=True`: the env's own (k, 84, 84) channels-first stack. Its values equal what VecFrameStack builds
  from the single frames (zero-padded after a reset), so VecFrameStack / VecTransposeImage are left out.

The SB3 side needs `stable_baselines3` and `gymnasium`, imported only when `sb3_vec_env` is called. The
translation from FastVecEnv's outputs to SB3's (`Sb3Frames`) has no such dependency.
"""
from __future__ import annotations

import numpy as np

from .env import N_ACTIONS, OBS_HW, FastVecEnv


class Sb3Frames:
    """FastVecEnv's outputs in SB3's VecEnv conventions.

    * obs: the (N, k, 84, 84) stack as is (stacked), or its single frame as (N, 84, 84, 1);
    * dones: terminated | truncated, as SB3's one `dones` array;
    * infos: `final_obs` becomes `terminal_observation` in the chosen layout, and `episode` is dropped, since
      SB3's VecMonitor writes its own; `TimeLimit.truncated` and the game fields stay."""

    def __init__(self, venv: FastVecEnv, stacked: bool):
        self.venv = venv
        self.stacked = bool(stacked)
        self.shape = (venv.k, OBS_HW, OBS_HW) if self.stacked else (OBS_HW, OBS_HW, 1)
        if not self.stacked and venv.k != 1:
            raise ValueError("single-frame SB3 observations need a FastVecEnv with frame_stack=1")

    def obs(self, o: np.ndarray) -> np.ndarray:
        return o if self.stacked else o[:, 0, :, :, None]

    def terminal(self, fin: np.ndarray) -> np.ndarray:
        return fin if self.stacked else fin[0][:, :, None]

    def reset(self) -> np.ndarray:
        return self.obs(self.venv.reset())

    def step_wait(self):
        o, rew, term, trunc, infos = self.venv.step_wait()
        for info in infos:
            fin = info.pop("final_obs", None)
            if fin is not None:
                info["terminal_observation"] = self.terminal(fin)
                info.pop("episode", None)
        return self.obs(o), rew, term | trunc, infos


def sb3_vec_env(level="1-1", n_envs=8, seed=0, stack_in_cpp=False, **kw):
    """An SB3 `VecEnv` of `n_envs` FastVecEnv envs (the reference's sb3_vec_env, sb3.py:10-71).

    `stack_in_cpp=False` gives single frames (the env runs with frame_stack=1; a `frame_stack` keyword is
    ignored, as in the reference); `stack_in_cpp=True` gives the env's (frame_stack, 84, 84) stacks. Other
    keywords go to FastVecEnv (sticky, noop_max, max_steps, maxpool, skip, rom_mode, rom, device, ...)."""
    try:
        from gymnasium import spaces
        from stable_baselines3.common.vec_env.base_vec_env import VecEnv
    except ImportError as e:
        raise ImportError("sb3_vec_env needs stable-baselines3 and gymnasium (pip install stable-baselines3)") from e

    k = kw.pop("frame_stack", 4)
    if not stack_in_cpp:
        k = 1

    class FastMarioSb3VecEnv(VecEnv):
        """FastVecEnv's envs behind SB3's VecEnv interface; per-env attribute access is not supported (the envs
        are one batched GPU object), so the attribute and method hooks answer None for every env."""

        def __init__(self):
            self.core = Sb3Frames(FastVecEnv(level, n_envs, seed=seed, frame_stack=k, **kw), stack_in_cpp)
            super().__init__(n_envs, spaces.Box(0, 255, self.core.shape, np.uint8), spaces.Discrete(N_ACTIONS))

        def reset(self):
            return self.core.reset()

        def step_async(self, actions):
            self.core.venv.step_async(actions)

        def step_wait(self):
            return self.core.step_wait()

        def close(self):
            self.core.venv.close()

        def _envs(self, indices):
            if indices is None:
                return list(range(self.num_envs))
            return [indices] if isinstance(indices, int) else list(indices)

        def get_attr(self, attr_name, indices=None):
            return [None for _ in self._envs(indices)]

        def set_attr(self, attr_name, value, indices=None):
            return None

        def env_method(self, method_name, *method_args, indices=None, **method_kwargs):
            return [None for _ in self._envs(indices)]

        def env_is_wrapped(self, wrapper_class, indices=None):
            return [False for _ in self._envs(indices)]

        def seed(self, seed=None):
            return [None for _ in range(self.num_envs)]

    return FastMarioSb3VecEnv()
