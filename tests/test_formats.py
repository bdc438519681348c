"""On-disk formats through the C library (no GPU needed): the reference's
deployed policy assets/navigation.bin (NAVPOL1, deployment.hpp:142-205) and
the checkpoint it was exported from (PPOFIX1 version 6, main.mm:978-994),
both unchanged copies of the reference's assets in tests/golden/."""
import os
import shutil

import numpy as np
import pytest

from mdnav import MdnError, abi, formats
from oracle_lib import GOLDEN, oracle, ptr, ref, ref_available

NAVPOL = os.path.join(GOLDEN, "navigation.bin")
CKPT = os.path.join(GOLDEN, "guided-table-memory.bin.best")
F = np.float32


def test_navigation_policy_metadata_and_provenance():
    meta, w, h = formats.read_navigation_policy(NAVPOL)
    assert (int(meta["version"]), int(meta["observation_count"]), int(meta["hidden_count"]),
            int(meta["action_count"]), int(meta["policy_mode"]), int(meta["weight_count"])) == (1, 184, 64, 4, 17, 12104)
    assert float(meta["max_speed_mps"]) == F(1.5) and int(meta["memory_frames"]) == 8
    assert int(meta["body_frame"]) == 0x00554C46  # "FLU\0"
    # the documented export: source FNV64 1d991b0048dec80a (docs/BENCHMARKS.md:94)
    assert h == 0x1D991B0048DEC80A
    assert formats.fnv1a64_file(CKPT) == h
    assert np.all(np.isfinite(w)) and w.size == 12104


def test_checkpoint_header_and_exported_actor():
    hd, actor = formats.read_checkpoint(CKPT)
    assert hd["magic"] == b"PPOFIX1" and int(hd["version"]) == 6
    assert (int(hd["actor_count"]), int(hd["critic_count"]), int(hd["horizon"]), int(hd["n"])) == (12104, 2177, 32, 128)
    assert (int(hd["family"]), int(hd["base_seed"]), int(hd["completed_rollouts"]), int(hd["optimizer_step"])) == \
        (5, 42, 1090, 34880)
    c = hd["config"]
    assert int(c["geometry_memory"]) == 1 and float(c["speed"]) == F(1.5) and float(c["distance"]) == F(4.0)
    # navigation.bin holds this checkpoint's actor unchanged
    assert np.array_equal(actor, formats.read_navigation_policy(NAVPOL)[1])
    assert os.path.getsize(CKPT) == 136 + 4 * (3 * 12104 + 3 * 2177) + 128 * (68 + 184 + 676 + 8 * 320 * 4 + 8 * 12 * 4 + 8 * 4 * 4)


def test_navigation_policy_write_round_trip(tmp_path):
    meta, w, h = formats.read_navigation_policy(NAVPOL)
    out = tmp_path / "copy.bin"
    formats.write_navigation_policy(out, w, meta, h)
    assert out.read_bytes() == open(NAVPOL, "rb").read()


@pytest.mark.parametrize("damage", ["magic", "truncated", "trailing", "nan_weight", "metadata"])
def test_navigation_policy_rejects_damaged_files(tmp_path, damage):
    data = bytearray(open(NAVPOL, "rb").read())
    if damage == "magic":
        data[0:8] = b"NAVPOL2\0"
    elif damage == "truncated":
        data = data[:-3]
    elif damage == "trailing":
        data += b"\0"
    elif damage == "nan_weight":
        data[64 + 400:64 + 404] = np.array([np.nan], F).tobytes()
    elif damage == "metadata":
        data[8 + 16:8 + 20] = np.array([13], np.uint32).tobytes()  # policy mode 13
    p = tmp_path / "bad.bin"
    p.write_bytes(bytes(data))
    with pytest.raises(MdnError):
        formats.read_navigation_policy(p)


def test_checkpoint_rejects_unknown_versions(tmp_path):
    data = bytearray(open(CKPT, "rb").read())
    data[8:12] = np.array([11], np.uint32).tobytes()
    p = tmp_path / "v11.bin"
    p.write_bytes(bytes(data))
    with pytest.raises(MdnError):
        formats.read_checkpoint(p)


def deployment_probe_observation(sample):
    """main.mm:1003-1018: the export's eight probe observations."""
    obs = np.zeros(184, F)
    i = np.arange(160)
    obs[:160] = (F(0.20) + F(0.01) * ((i * 13 + sample * 7) % 70).astype(F)).astype(F)
    c = 160
    angle = F(-0.7) + F(0.2) * F(sample)
    obs[c + 0] = np.cos(np.float64(angle))
    obs[c + 1] = np.sin(np.float64(angle))
    obs[c + 2] = 0.1
    obs[c + 3] = F(0.3) + F(0.04) * F(sample)
    obs[c + 4:c + 21] = [0.1, -0.05, 0.02, 0.01, -0.02, 0.03, 0.0, 0.0, 1.0, 0.05, -0.03, 0.0, 0.02, 0.01, 0.02,
                         -0.01, 0.0]
    obs[181:184] = [0.08, -0.04, 0.02]
    return obs


@pytest.mark.skipif(not ref_available(184), reason="oracle/_ref not built")
def test_deployment_probe_parity():
    """main.mm:1024-1047: the exported actor's means on the eight probe
    observations match fixed_ppo::actor_forward within 2e-5 (the oracle here,
    the reference's ppo.hpp built at 184 inputs there)."""
    w = formats.read_navigation_policy(NAVPOL)[1]
    obs = np.stack([deployment_probe_observation(k) for k in range(8)])
    h = np.zeros((8, 64), F)
    m = np.zeros((8, 4), F)
    oracle().orc_actor_forward_batch(ptr(w), ptr(obs), 184, 64, 8, ptr(h), ptr(m))
    worst = 0.0
    for k in range(8):
        rh, rm = np.zeros(64, F), np.zeros(4, F)
        ref(184).ref_actor_forward(ptr(w), ptr(obs[k]), ptr(rh), ptr(rm))
        worst = max(worst, float(np.abs(rm - m[k]).max()))
    assert worst < 2e-5, worst


# ---------------------------------------------------------------- NAVWID4
def test_wide_policy_export_matches_reference_loader(tmp_path):
    """navigation_export_wide.py's export of the trained guided checkpoint
    (184-64-4) as NAVWID4, read back here and by the reference's own
    WideNavigationPolicy::load (navigation_wide_deployment.hpp, built into
    oracle/_ref): metadata, camera contract, weights (the checkpoint's
    actor) and the FNV-1a provenance agree, and the reference's raw_mean on
    random observations matches the oracle's forward of the same actor."""
    import ctypes
    from oracle_lib import ref, ref_available
    # the trained checkpoint was saved in training mode 0, which the export
    # refuses (navigation_export_wide.py:22-24); a copy with its config mode
    # set to 22 (training through the deployed map) is exported
    src = os.path.join(GOLDEN, "guided-table-memory.bin.best")
    with pytest.raises(ValueError):
        formats.export_wide_policy(src, str(tmp_path / "refused.bin"))
    data = bytearray(open(src, "rb").read())
    data[56:60] = np.uint32(22).tobytes()
    ckpt = str(tmp_path / "mode22.bin")
    open(ckpt, "wb").write(bytes(data))
    out = str(tmp_path / "wide.bin")
    record = formats.export_wide_policy(ckpt, out)
    meta, cam, w, h = formats.read_wide_policy(out)
    import hashlib
    import json
    assert json.load(open(out + ".json")) == record
    assert record["source_fnv1a64"] == h and record["actor_hidden"] == 64 and record["bytes"] == os.path.getsize(out)
    assert record["nav_sha256"] == hashlib.sha256(open(out, "rb").read()).hexdigest()
    assert record["source_critic_parameters"] == 2177 and record["sensor_profile"] == 1
    _, actor = formats.read_checkpoint(ckpt)
    assert int(meta["version"]) == 4 and int(meta["hidden_count"]) == 64 and w.size == 189 * 64 + 8
    assert np.array_equal(w, actor) and h == formats.fnv1a64_file(ckpt)
    assert int(cam["profile_id"]) == 1 and abs(float(cam["tan_v"]) - 0.75) < 1e-7
    if not ref_available():
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    rng = np.random.default_rng(11)
    obs = rng.uniform(0, 1, (16, 184)).astype(np.float32)
    obs[:, 181:] = rng.normal(0, 0.5, (16, 3))
    m2, c2 = np.zeros((), abi.NAV_POLICY_META), np.zeros((), abi.SENSOR_CONTRACT)
    h2 = ctypes.c_uint64()
    means = np.zeros((16, 4), np.float32)
    assert ref().ref_navwid_load(out.encode(), ptr(m2), ptr(c2), ctypes.byref(h2), ptr(obs), 16, ptr(means)) == 1
    assert m2.tobytes() == meta.tobytes() and c2.tobytes() == cam.tobytes() and h2.value == h
    hid = np.zeros((16, 64), np.float32)
    mine = np.zeros((16, 4), np.float32)
    oracle().orc_actor_forward_batch(ptr(w), ptr(obs), 184, 64, 16, ptr(hid), ptr(mine))
    assert np.abs(mine - means).max() < 1e-5


def test_wide_policy_round_trip_and_rejections(tmp_path):
    """A 184-256-4 actor written and read back bit for bit; the reader
    rejects what WideNavigationPolicy::load rejects."""
    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.1, 189 * 256 + 8).astype(np.float32)
    meta = formats.default_navigation_metadata(2.0)
    meta["version"], meta["hidden_count"], meta["weight_count"] = 4, 256, w.size
    cam = np.zeros((), abi.SENSOR_CONTRACT)
    cam["profile_id"], cam["tan_h"], cam["tan_v"], cam["min_range_m"], cam["max_range_m"] = 1, 1.0, 0.75, 0.03, 12.0
    path = str(tmp_path / "w.bin")
    from mdnav.native import lib
    assert lib().mdn_navwid_write(path.encode(), ptr(meta), ptr(cam), ptr(w), w.size, 77) == 0
    m2, c2, w2, h2 = formats.read_wide_policy(path)
    assert np.array_equal(w2, w) and h2 == 77 and m2.tobytes() == meta.tobytes()
    data = open(path, "rb").read()
    for bad in (data + b"\0", b"NAVWID5\0" + data[8:], data[:100]):
        open(path, "wb").write(bad)
        with pytest.raises(Exception):
            formats.read_wide_policy(path)
    w[3] = np.nan
    assert lib().mdn_navwid_write(path.encode(), ptr(meta), ptr(cam), ptr(w), w.size, 77) != 0
    w[3] = 0.0
    meta["policy_mode"] = 2
    assert lib().mdn_navwid_write(path.encode(), ptr(meta), ptr(cam), ptr(w), w.size, 77) != 0


def test_wide_policy_export_rejections(tmp_path):
    """navigation_export_wide.py:27-40: a truncated actor/critic payload, a
    non-finite actor weight and a sidecar naming another architecture or
    camera are refused."""
    import json
    data = bytearray(open(os.path.join(GOLDEN, "guided-table-memory.bin.best"), "rb").read())
    data[56:60] = np.uint32(22).tobytes()
    actor_count, critic_count = np.frombuffer(bytes(data[12:20]), np.uint32)
    end = 136 + 4 * int(actor_count + critic_count)
    cases = {"truncated": bytes(data[:end - 4]), "nan": None}
    bad = bytearray(data)
    bad[136 + 40:136 + 44] = np.float32(np.nan).tobytes()
    cases["nan"] = bytes(bad)
    for name, blob in cases.items():
        src = str(tmp_path / (name + ".bin"))
        open(src, "wb").write(blob)
        with pytest.raises(ValueError):
            formats.export_wide_policy(src, str(tmp_path / (name + ".out")))
    src = str(tmp_path / "ok.bin")
    open(src, "wb").write(bytes(data[:end]))  # the actor/critic prefix alone is enough
    formats.export_wide_policy(src, str(tmp_path / "ok.out"))
    for sidecar in ({"actor_obs_dim": 184, "actor_hidden_dim": 256, "sensor_profile": "legacy"},
                    {"actor_obs_dim": 184, "actor_hidden_dim": 64, "sensor_profile": "native"}):
        open(src + ".train.json", "w").write(json.dumps(sidecar))
        with pytest.raises(ValueError):
            formats.export_wide_policy(src, str(tmp_path / "side.out"))
    open(src + ".train.json", "w").write(json.dumps({"actor_obs_dim": 184, "actor_hidden_dim": 64,
                                                      "sensor_profile": "legacy"}))
    formats.export_wide_policy(src, str(tmp_path / "side.out"))
