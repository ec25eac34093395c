"""Host-side API and boundary checks that need no GPU (mirrors the reference's tests/test_api.py)."""
import ctypes
import os
import sys
import re
import subprocess

import numpy as np
import pytest
from conftest import HAVE_GPU, ROOT

import fast_mario_env_amd as fme
from fast_mario_env_amd import _native, rom
from build_roms import MODES, rom_path

HEADER = os.path.join(ROOT, "include", "mario_hip.h")


def test_decode_level():
    """Known answers of the reference's test_api.py:10-18."""
    assert fme.decode_level("1-1") == (1, 1, 1)
    assert fme.decode_level("1-2") == (1, 2, 3)
    assert fme.decode_level((4, 4)) == (4, 4, 5)
    assert fme.decode_level("3-2") == (3, 2, 2)
    assert fme.decode_level("8-4") == (8, 4, 4)
    for bad in ("0-1", "9-1", "1-5", "x"):
        with pytest.raises(ValueError):
            fme.decode_level(bad)
    assert len(fme.ALL_LEVELS) == 32 and fme.ALL_LEVELS[0] == "1-1" and fme.ALL_LEVELS[-1] == "8-4"


def test_missing_rom_message(tmp_path, monkeypatch):
    monkeypatch.setenv(fme.ROM_ENV_VAR, str(tmp_path / "nope.nes"))
    with pytest.raises(fme.RomNotFoundError, match="does not ship a ROM"):
        fme.find_rom()


def test_rom_lookup_order(tmp_path, monkeypatch):
    a, b = tmp_path / "a.nes", tmp_path / "b.nes"
    data = open(rom_path("vanilla"), "rb").read()
    a.write_bytes(data)
    b.write_bytes(data)
    monkeypatch.setenv(fme.ROM_ENV_VAR, str(b))
    assert fme.find_rom(a) == str(a)            # rom_path wins over the environment variable
    assert fme.find_rom() == str(b)
    assert fme.load_rom() == data
    with pytest.raises(ValueError):
        fme.find_rom(a, rom_mode="nope")


def test_bad_rom_rejected(tmp_path):
    p = tmp_path / "bad.nes"
    p.write_bytes(b"not a rom" * 100)
    with pytest.raises(ValueError, match="iNES"):
        fme.load_rom(p)
    good = bytearray(open(rom_path("vanilla"), "rb").read())
    good[6] |= 0x10                               # mapper 1
    with pytest.raises(ValueError, match="unsupported"):
        fme.check_rom(bytes(good))
    with pytest.raises(ValueError, match="truncated"):
        fme.check_rom(bytes(open(rom_path("vanilla"), "rb").read()[:30000]))


def test_rom_file_table():
    assert rom.ROM_FILES["vanilla"] == "super-mario-bros.nes"
    assert set(rom.ROM_FILES) == set(MODES)


def test_rng_state_words():
    st = np.random.default_rng(5).bit_generator.state
    w = fme.rng_state(5)
    assert (w[0] << 64 | w[1]) == st["state"]["state"] and (w[2] << 64 | w[3]) == st["state"]["inc"]


def _declared_symbols():
    return sorted(set(re.findall(r"\b(mh_\w+)\s*\(", open(HEADER).read())))


def test_library_exports_header():
    """libmario_hip.so loads without a GPU and exports every entry point include/mario_hip.h declares."""
    L = ctypes.CDLL(_native.lib_path())
    syms = _declared_symbols()
    assert len(syms) >= 25
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    L.mh_state_bytes.restype = ctypes.c_int64
    assert L.mh_state_bytes() > 4384


def test_bindings_cover_header():
    src = open(os.path.join(ROOT, "fast-mario-env_amd", "fast_mario_env_amd", "_native.py")).read()
    for s in _declared_symbols():
        assert s in src, f"{s} has no ctypes binding"


def test_create_roms_validates_before_the_gpu():
    """mh_create_roms rejects ROMs that differ in PRG (per-env rom_mode variants differ in CHR only) and a
    bad env ROM index, with a message, before it touches a device."""
    L = ctypes.CDLL(_native.lib_path())
    L.mh_create_roms.restype = ctypes.c_void_p
    L.mh_last_error.restype = ctypes.c_char_p
    import fuzz
    n = 2
    lv = np.array([1, 1, 1] * n, np.int32)
    lut = fme.gray_lut()
    rng = np.zeros(6 * n, np.uint64)
    P = ctypes.c_void_p

    def create(roms, env_rom):
        blob = np.frombuffer(b"".join(roms), np.uint8).copy()
        lens = np.array([len(b) for b in roms], np.int64)
        er = np.array(env_rom, np.int32)
        return L.mh_create_roms(P(blob.ctypes.data), P(lens.ctypes.data), len(roms), P(er.ctypes.data), n,
                                P(lv.ctypes.data), P(lut.ctypes.data), 4, 2000, ctypes.c_double(0.0), 0, 0, 4,
                                P(rng.ctypes.data), 0)
    mini = open(rom_path("vanilla"), "rb").read()
    assert not create([mini, fuzz.program_rom(0)], [0, 1])
    assert b"share PRG" in L.mh_last_error()
    assert not create([mini, open(rom_path("pixel"), "rb").read()], [0, 2])
    assert b"out of range" in L.mh_last_error()
    with pytest.raises(ValueError, match="rom modes"):
        fme.HipVecEnv("1-1", 3, rom_mode=["vanilla", "pixel"])
    with pytest.raises(ValueError, match="at most 4"):
        fme.HipVecEnv("1-1", 5, rom_mode=["vanilla", "pixel", "downsample", "rectangle", "other"])


def test_create_rejects_more_envs_than_32bit_offsets_address():
    """The console memory (4,384 rows of np bytes) is addressed with 32-bit offsets from its base: both
    creators refuse more than 979,648 envs, with a message, before they touch a device."""
    L = ctypes.CDLL(_native.lib_path())
    L.mh_create_roms.restype = ctypes.c_void_p
    L.mh_raw_create.restype = ctypes.c_void_p
    L.mh_last_error.restype = ctypes.c_char_p
    P = ctypes.c_void_p
    n = 979_649
    mini = open(rom_path("vanilla"), "rb").read()
    blob = np.frombuffer(mini, np.uint8).copy()
    lens = np.array([len(mini)], np.int64)
    lv = np.ones(3 * n, np.int32)
    rng = np.zeros(6 * n, np.uint64)
    lut = fme.gray_lut()
    assert not L.mh_create_roms(P(blob.ctypes.data), P(lens.ctypes.data), 1, None, n, P(lv.ctypes.data),
                                P(lut.ctypes.data), 4, 2000, ctypes.c_double(0.0), 0, 0, 4, P(rng.ctypes.data), 0)
    assert b"too many envs" in L.mh_last_error()
    assert not L.mh_raw_create(P(blob.ctypes.data), ctypes.c_int64(len(mini)), n, 0)
    assert b"too many consoles" in L.mh_last_error()


@pytest.mark.parametrize("value", ["3", "32", "0", "x"])
def test_raw_create_rejects_bad_consoles_per_wave(monkeypatch, value):
    """MH_RAW_CONSOLES_PER_WAVE (k_raw's consoles per wave, a power of two up to 16) is checked at creation,
    before the device is touched."""
    L = ctypes.CDLL(_native.lib_path())
    L.mh_raw_create.restype = ctypes.c_void_p
    L.mh_last_error.restype = ctypes.c_char_p
    monkeypatch.setenv("MH_RAW_CONSOLES_PER_WAVE", value)
    mini = open(rom_path("vanilla"), "rb").read()
    blob = np.frombuffer(mini, np.uint8).copy()
    assert not L.mh_raw_create(ctypes.c_void_p(blob.ctypes.data), ctypes.c_int64(len(mini)), 4, 0)
    assert b"MH_RAW_CONSOLES_PER_WAVE must be" in L.mh_last_error()


@pytest.mark.skipif(HAVE_GPU, reason="checks the no-GPU error path")
def test_no_cpu_fallback():
    """Without a GPU the product raises; there is no silent CPU path."""
    with pytest.raises(RuntimeError, match="GPU"):
        fme.HipVecEnv("1-1", 2, rom=open(rom_path("vanilla"), "rb").read())


def test_resize_kernel_has_no_fma(tmp_path):
    """The INTER_AREA float sums must not be contracted into FMAs (bit-exactness with the reference's
    -ffp-contract=off build): compile the device code to gfx950 assembly and inspect the obs code (k_step's
    obs_tail, a function of its own, and the kernels for reset-cache entries and images)."""
    src = os.path.join(ROOT, "fast-mario-env_amd", "csrc", "mario_hip.hip")
    out = tmp_path / "dev.s"
    sys.path.insert(0, os.path.join(ROOT, "fast-mario-env_amd"))
    import build_native                                  # the library's own flags
    flags = [f for f in build_native.FLAGS if f not in ("-shared", "-fPIC", "-Wall")]
    assert "-ffp-contract=off" in flags
    cmd = ["hipcc", "--offload-arch=gfx950", "--cuda-device-only", "-S", *flags, src, "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = out.read_text()
    checked = 0
    for name in ("obs_tail", "k_small_obs", "k_resize_images"):
        m = re.search(rf"^(_Z\w*{name}\w*):[^\n]*$(.*?)^\s*(s_endpgm|s_setpc_b64)", asm, re.S | re.M)
        assert m, name
        body = m.group(2)
        assert "v_mul_f32" in body and "v_add_f32" in body
        assert not re.search(r"\bv_(fma|fmac|mac|mad|pk_fma)\w*_f32", body), name
        checked += 1
    assert checked == 3


class _FakeVec:
    """Stands in for FastVecEnv in the SB3 translation tests: fixed outputs, two envs, env 1 ends its episode."""

    def __init__(self, k):
        self.k = k
        self.o = np.arange(2 * k * 84 * 84, dtype=np.int64).astype(np.uint8).reshape(2, k, 84, 84)
        self.fin = (255 - self.o[1]).copy()

    def reset(self):
        return self.o

    def step_wait(self):
        infos = [{"x_pos": 40}, {"x_pos": 41, "final_obs": self.fin, "TimeLimit.truncated": True,
                                  "episode": {"r": 1.0, "l": 5}}]
        return self.o, np.array([0.5, 1.0], np.float32), np.array([False, False]), np.array([False, True]), infos


@pytest.mark.parametrize("stacked", [False, True])
def test_sb3_translation(stacked):
    """sb3.py:38-49 of the reference: channels-last single frames or the stack as is, dones = term | trunc,
    final_obs renamed terminal_observation in the same layout, episode dropped (VecMonitor writes its own)."""
    k = 4 if stacked else 1
    venv = _FakeVec(k)
    core = fme.Sb3Frames(venv, stacked)
    o = core.reset()
    assert core.shape == ((4, 84, 84) if stacked else (84, 84, 1))
    assert o.shape == (2,) + core.shape
    assert np.array_equal(o, venv.o if stacked else venv.o[:, 0, :, :, None])
    o, r, d, infos = core.step_wait()
    assert d.tolist() == [False, True] and r.tolist() == [0.5, 1.0]
    assert "terminal_observation" not in infos[0] and infos[0]["x_pos"] == 40
    t = infos[1]["terminal_observation"]
    assert np.array_equal(t, venv.fin if stacked else venv.fin[0][:, :, None])
    assert "episode" not in infos[1] and "final_obs" not in infos[1] and infos[1]["TimeLimit.truncated"]
    if not stacked:
        with pytest.raises(ValueError, match="frame_stack=1"):
            fme.Sb3Frames(_FakeVec(4), False)


def test_sb3_adapter_without_sb3():
    """sb3_vec_env needs stable-baselines3 and gymnasium, which this image lacks: the call says so."""
    try:
        import gymnasium  # noqa: F401
        import stable_baselines3  # noqa: F401
        pytest.skip("stable-baselines3 is installed")
    except ImportError:
        pass
    with pytest.raises(ImportError, match="stable-baselines3"):
        fme.sb3_vec_env("1-1", 2)
