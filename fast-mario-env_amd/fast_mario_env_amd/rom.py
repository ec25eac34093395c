"""Where the Super Mario Bros ROM comes from, what an acceptable image looks like, and level names.

Interface of the reference's src/fast_mario_env/rom.py (lookup order, file names, header rules and the
world/stage -> area rule are kept; the code is this package's own):

* No ROM is bundled. `find_rom` tries, in order, the explicit ``rom_path`` argument, the
  ``FAST_MARIO_ENV_ROM`` environment variable, and the ``_roms`` directory of an installed
  gym-super-mario-bros distribution (located with importlib's finder; the package is never imported).
  An explicit path that does not exist is an error, not a reason to keep looking.
* `check_rom` accepts iNES NROM images only: mapper 0, one or two 16 KB PRG banks, one 8 KB CHR bank.
* `decode_level` maps "w-s" to gym-super-mario-bros' (world, stage, area) target.
"""
from __future__ import annotations

import importlib.util
import os
from dataclasses import dataclass
from typing import Iterator, Optional, Tuple

ROM_ENV_VAR = "FAST_MARIO_ENV_ROM"

# gym-super-mario-bros ships one file per ROM mode; these names are part of the lookup interface
ROM_FILES = {
    "vanilla": "super-mario-bros.nes",
    "downsample": "super-mario-bros-downsample.nes",
    "pixel": "super-mario-bros-pixel.nes",
    "rectangle": "super-mario-bros-rectangle.nes",
}

_HOW_TO_PROVIDE = "\n".join([
    "This package does not ship a ROM; it reads yours. Any one of these works:",
    "  - pass rom_path='.../super-mario-bros.nes' to the env constructor;",
    f"  - export {ROM_ENV_VAR}=.../super-mario-bros.nes;",
    "  - have gym-super-mario-bros installed: the ROM files it carries are found on disk.",
    "Only iNES images with mapper 0 (NROM), like the original Super Mario Bros cartridge, can run.",
])


class RomNotFoundError(FileNotFoundError):
    """No usable ROM file was found (or an explicitly given path does not exist)."""


def _installed_rom_dir() -> Optional[str]:
    """`_roms` directory of an installed gym_super_mario_bros package, without importing it."""
    spec = importlib.util.find_spec("gym_super_mario_bros")
    locations = list(spec.submodule_search_locations or []) if spec is not None else []
    return os.path.join(locations[0], "_roms") if locations else None


def _explicit_sources(rom_path) -> Iterator[Tuple[str, str]]:
    """(where it came from, path) for the sources that must exist once given."""
    if rom_path is not None:
        yield "rom_path", os.fspath(rom_path)
    env_value = os.environ.get(ROM_ENV_VAR)
    if env_value:
        yield ROM_ENV_VAR, env_value


def find_rom(rom_path=None, rom_mode: str = "vanilla") -> str:
    """Path of the ROM for `rom_mode`: rom_path, then $FAST_MARIO_ENV_ROM, then gym-super-mario-bros' files."""
    if rom_mode not in ROM_FILES:
        raise ValueError(f"unknown rom_mode {rom_mode!r}; expected one of {sorted(ROM_FILES)}")
    for origin, raw in _explicit_sources(rom_path):
        path = os.path.expanduser(raw)
        if os.path.isfile(path):
            return path
        raise RomNotFoundError(f"{origin} is set to {path!r}, but no such file exists.\n{_HOW_TO_PROVIDE}")
    rom_dir = _installed_rom_dir()
    if rom_dir:
        path = os.path.join(rom_dir, ROM_FILES[rom_mode])
        if os.path.isfile(path):
            return path
    raise RomNotFoundError(f"Could not locate a Super Mario Bros ROM.\n{_HOW_TO_PROVIDE}")


@dataclass(frozen=True)
class INesHeader:
    """The fields of a 16-byte iNES header this package cares about."""
    prg_banks: int     # 16 KB units
    chr_banks: int     # 8 KB units
    mapper: int

    @classmethod
    def parse(cls, data: bytes, name: str) -> "INesHeader":
        if len(data) < 16 or bytes(data[:4]) != b"NES\x1a":
            raise ValueError(f"{name}: the file does not start with an iNES header")
        return cls(prg_banks=data[4], chr_banks=data[5], mapper=(data[7] & 0xF0) | (data[6] >> 4))

    @property
    def payload_bytes(self) -> int:
        return self.prg_banks * 0x4000 + self.chr_banks * 0x2000


def check_rom(data: bytes, name: str = "ROM") -> None:
    """Raise ValueError unless `data` is a complete iNES NROM image (mapper 0, 16 or 32 KB PRG, 8 KB CHR)."""
    h = INesHeader.parse(data, name)
    if h.mapper != 0 or h.prg_banks not in (1, 2) or h.chr_banks != 1:
        raise ValueError(f"{name}: unsupported cartridge (mapper {h.mapper}, {h.prg_banks} PRG bank(s) of 16 KB, "
                         f"{h.chr_banks} CHR bank(s) of 8 KB); only NROM images can run")
    if len(data) < 16 + h.payload_bytes:
        raise ValueError(f"{name}: truncated image ({len(data)} bytes, the header promises {16 + h.payload_bytes})")


def load_rom(rom_path=None, rom_mode: str = "vanilla") -> bytes:
    """The bytes of the ROM find_rom() picks, checked with check_rom()."""
    path = find_rom(rom_path, rom_mode)
    with open(path, "rb") as fh:
        data = fh.read()
    check_rom(data, path)
    return data


ALL_LEVELS = tuple(f"{world}-{stage}" for world in range(1, 9) for stage in range(1, 5))

# Worlds whose second stage is preceded by a separate intro area (the pipe scene), which shifts the area
# number of every later stage of that world by one.
_WORLDS_WITH_INTRO_AREA = frozenset({1, 2, 4, 7})


def decode_level(level) -> Tuple[int, int, int]:
    """"w-s" or (w, s) -> (world, stage, area)."""
    if isinstance(level, str):
        parts = level.split("-")
        if len(parts) != 2 or not all(p.strip().lstrip("+-").isdigit() for p in parts):
            raise ValueError(f"level must look like '1-1', got {level!r}")
        world, stage = int(parts[0]), int(parts[1])
    else:
        world, stage = (int(v) for v in level)
    if world not in range(1, 9) or stage not in range(1, 5):
        raise ValueError(f"level {level!r} out of range (worlds 1-8, stages 1-4)")
    area = stage + (1 if world in _WORLDS_WITH_INTRO_AREA and stage > 1 else 0)
    return world, stage, area
