"""fast_mario_env_amd: bit-exact batched Super Mario Bros envs on one AMD MI355X (gfx950).

    from fast_mario_env_amd import HipVecEnv, FastVecEnv, RawNES, sb3_vec_env

The env step is HIP code built for gfx950 (csrc/ -> libmario_hip.so, C ABI in include/mario_hip.h);
this package is the host side that mirrors the reference's Python API (src/fast_mario_env).
"""
from .env import (CANON_BYTES, INFO_FIELDS, INFO_KEYS, N_ACTIONS, OBS_HW, PALETTE, SIMPLE_MOVEMENT, CudaVecEnv,
                  FastVecEnv, HipRawNES, HipVecEnv, MonitorCSV, RawNES, gray_lut, palette_rgb, resize_area,
                  rng_state)
from .sb3 import Sb3Frames, sb3_vec_env
from .rom import ALL_LEVELS, ROM_ENV_VAR, ROM_FILES, RomNotFoundError, check_rom, decode_level, find_rom, load_rom

__version__ = "0.1.0"

__all__ = ["HipVecEnv", "CudaVecEnv", "FastVecEnv", "HipRawNES", "RawNES", "MonitorCSV", "palette_rgb", "gray_lut",
           "rng_state", "resize_area", "find_rom", "load_rom", "check_rom", "decode_level", "RomNotFoundError",
           "ROM_ENV_VAR", "ROM_FILES", "ALL_LEVELS", "OBS_HW", "N_ACTIONS", "SIMPLE_MOVEMENT", "INFO_FIELDS",
           "INFO_KEYS", "PALETTE", "CANON_BYTES", "sb3_vec_env", "Sb3Frames", "__version__"]
