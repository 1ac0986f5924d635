"""Host-side pieces of the trainer: the reproduced System.Random stream, the cosine schedule, temperature
fitting, the calibration sample and the written config (no GPU)."""
import json
import math
import os
import shutil

import numpy as np
import pytest

from laya_amd.batch import TrainingItem
from laya_amd.calibration import CalibrationSample, clamp_temperature, fit, fit_one, temperature_bucket
from laya_amd.netrandom import DotNetRandom, gaussian, trainer_shuffle
from laya_amd.trainer import CosineSchedule, TrainerOptions, build_config, calibration_sample, write_temperatures

from fixtures import TINY


def test_dotnet_random_known_answers():
    """Values .NET's seeded System.Random is documented and widely quoted to produce (the same on every
    .NET version, since seeded instances keep the legacy subtractive generator)."""
    assert DotNetRandom(0).next_double() == 0.7262432699679598
    assert DotNetRandom(0).next() == 1559595546
    assert DotNetRandom(1).next_double() == pytest.approx(0.248668584157093, abs=1e-15)
    assert DotNetRandom(42).next() == 1434747710


def test_dotnet_random_structure():
    """Next(n) truncates Sample()·n, Next(lo, hi) offsets it, a saved state continues the same stream,
    and the outputs are uniform in [0, 1)."""
    a, b = DotNetRandom(7), DotNetRandom(7)
    for n in (1, 2, 10, 97, 2 ** 31 - 1):
        d = b.next_double()
        assert a.next(n) == int(d * n)
    c = DotNetRandom.from_state(a.state())
    assert [a.next() for _ in range(100)] == [c.next() for _ in range(100)]
    r, q = DotNetRandom(-5), DotNetRandom(5)  # |seed| is used
    assert [r.next() for _ in range(5)] == [q.next() for _ in range(5)]
    g = DotNetRandom(11)
    u = np.array([g.next_double() for _ in range(20000)])
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.01 and abs(u.var() - 1 / 12) < 0.005
    with pytest.raises(ValueError):
        DotNetRandom(2 ** 31)


def test_shuffles_are_permutations_and_reproducible():
    items = list(range(50))
    trainer_shuffle(items, DotNetRandom(42))
    assert sorted(items) == list(range(50)) and items != list(range(50))
    again = list(range(50))
    trainer_shuffle(again, DotNetRandom(42))
    assert items == again
    span = list(range(50))
    DotNetRandom(42).shuffle_span(span)
    assert sorted(span) == list(range(50)) and span != items  # a different algorithm, a different order


def test_gaussian_draws_are_standard_normal():
    g = DotNetRandom(5)
    z = np.array([gaussian(g) for _ in range(40000)])
    assert abs(z.mean()) < 0.02 and abs(z.std() - 1) < 0.02
    assert abs(np.mean(z ** 4) - 3) < 0.15  # Gaussian kurtosis


def test_cosine_schedule_matches_pytorch():
    """The reference's CosineAnnealingLR(T_max = 3, eta_min = 1e-6) rates (TrainingTests.cs:59)."""
    s = CosineSchedule([0.1], 3, 1e-6)
    assert s.rates == [0.1]
    for want in (0.07500025, 0.025000750000000013, 1e-6):
        s.step()
        assert s.rates[0] == pytest.approx(want, abs=1e-12)
    assert CosineSchedule([0.1, 0.2], 3, 1e-6, step=2).rates[1] == pytest.approx(s.at(0.2, 2))


def _known_temperature_samples():
    """TrainingTests.cs:86-97: logits U[-4, 4) from System.Random(5), targets softmax(z / 2) in fp32."""
    r = DotNetRandom(5)
    samples = []
    for _ in range(400):
        z = np.array([r.next_double() * 8 - 4 for _ in range(4)], np.float32)
        t = (z / np.float32(2)).astype(np.float32)
        e = np.exp(t - t.max()).astype(np.float32)
        samples.append(CalibrationSample(0, z, (e / e.sum()).astype(np.float32)))
    return samples


def test_temperature_fitting_recovers_a_known_temperature():
    """TrainingTests.cs:84-104: T = 2 to three decimals; five samples are too few (1.0); a type with no
    samples gets 1.2; the 'choice:3-5' bucket is fitted too."""
    samples = _known_temperature_samples()
    assert fit_one(samples) == pytest.approx(2.0, abs=5e-4)
    assert fit_one(samples[:5]) == 1.0
    f = fit(samples, minimum_bucket_samples=30)
    assert f.by_type[0] == pytest.approx(2.0, abs=5e-4)
    assert f.by_type[2] == float(np.float32(1.2))
    assert f.by_bucket["choice:3-5"] == pytest.approx(2.0, abs=5e-4)
    assert f.samples_per_bucket == {"choice:3-5": 400}


def test_temperature_fit_other_temperatures_and_clamping():
    rng = np.random.default_rng(0)
    for t0, expect in ((0.7, 0.7), (3.3, 3.3), (9.0, 5.0), (0.1, 0.5)):
        samples = []
        for _ in range(60):
            z = rng.uniform(-4, 4, 5).astype(np.float32)
            e = np.exp(z / t0 - (z / t0).max())
            samples.append(CalibrationSample(1, z, (e / e.sum()).astype(np.float32)))
        assert fit(samples).by_type[1] == pytest.approx(expect, rel=1e-3), t0
    assert clamp_temperature(float("nan")) == 1.0
    assert [temperature_bucket(q, k) for q, k in ((0, 2), (1, 3), (2, 5), (0, 6), (1, 10), (2, 11), (3, 4))] == [
        "choice:2", "score:3-5", "noul:3-5", "choice:6-10", "score:6-10", "noul:11+", "noul:3-5"]


def test_calibration_sample_covers_every_question_type():
    """TrainingTests.cs:106-119: 1500 items, five questions per case in a fixed order; a stride would pick
    only choices, the seeded draw picks 100 items of every type, reproducibly, in item order."""
    types = [0, 2, 0, 1, 1]
    items = [TrainingItem(np.array([0]), np.array([0, 1]), types[i % 5], np.array([0.5, 0.5], np.float32))
             for i in range(1500)]
    sample = calibration_sample(items, TrainerOptions())
    assert len(sample) == 100
    assert sorted({i.question_type for i in sample}) == [0, 1, 2]
    again = calibration_sample(items, TrainerOptions())
    assert [id(i) for i in sample] == [id(i) for i in again]
    where = {id(item): k for k, item in enumerate(items)}
    positions = [where[id(i)] for i in sample]
    assert positions == sorted(positions)
    assert len(calibration_sample(items[:20], TrainerOptions())) == 2


def test_build_config_keeps_unknown_keys(tmp_path):
    src = tmp_path / "src"
    src.mkdir()
    with open(os.path.join(TINY, "rl_agent_config.json")) as f:
        base = json.load(f)
    base["future_key"] = {"kept": True}
    base["temperature_by_options"] = {"choice:2": 3.0}
    (src / "rl_agent_config.json").write_text(json.dumps(base))
    fitted = fit(_known_temperature_samples())
    cfg = build_config(str(src), TrainerOptions(model_name="m", trainable_encoder_layers=2), fitted, 128, None, 7, 2,
                       5400.0)
    assert cfg["future_key"] == {"kept": True}
    assert cfg["max_len"] == 128 and cfg["head_max_len"] == base["head_max_len"]
    assert cfg["fine_tuned"] is True and cfg["model_name"] == "m"
    assert cfg["temperature_by_options"] == {"choice:3-5": fitted.by_bucket["choice:3-5"]}  # replaced, not merged
    assert cfg["training"]["updates"] == 7 and cfg["training"]["epochs_completed"] == 2
    assert cfg["training"]["hours"] == 1.5 and cfg["training"]["trainable_encoder_layers"] == 2
    c2 = {}
    write_temperatures(c2, fitted)
    assert c2["temperature"][2] == float(np.float32(1.2))


def test_rolling_checkpoint_swap_survives_an_interruption(tmp_path):
    """The rolling checkpoint is written whole into a sibling directory and swapped in by renames; an
    interruption at any point leaves one complete checkpoint that resume picks up."""
    import json

    from laya_amd.trainer import STATE_FILE, _recover_rolling, _swap_in

    def make(d, epoch):
        os.makedirs(d, exist_ok=True)
        with open(os.path.join(d, "model.safetensors"), "w") as f:
            f.write(f"weights {epoch}")
        with open(os.path.join(d, STATE_FILE), "w") as f:
            json.dump({"next_epoch": epoch}, f)

    def epoch_of(d):
        a = open(os.path.join(d, "model.safetensors")).read().split()[1]
        with open(os.path.join(d, STATE_FILE)) as f:
            b = json.load(f)["next_epoch"]
        assert int(a) == b
        return b

    rolling = str(tmp_path / "checkpoint_latest")
    make(rolling + ".new", 1)
    _swap_in(rolling + ".new", rolling)
    assert epoch_of(rolling) == 1 and not os.path.exists(rolling + ".new")
    # Interrupted after the old checkpoint was retired, before the new one moved in: the staged one is whole.
    make(rolling + ".new", 2)
    os.rename(rolling, rolling + ".old")
    _recover_rolling(rolling)
    assert epoch_of(rolling) == 2
    # Interrupted while staging (no loop state yet): the retired checkpoint comes back.
    shutil.rmtree(rolling + ".old", ignore_errors=True)
    os.rename(rolling, rolling + ".old")
    os.makedirs(rolling + ".new")
    with open(os.path.join(rolling + ".new", "model.safetensors"), "w") as f:
        f.write("weights 3")
    _recover_rolling(rolling)
    assert epoch_of(rolling) == 2
    # A staged loop state cut short (present but not parseable) does not count as complete.
    shutil.rmtree(rolling + ".new", ignore_errors=True)
    make(rolling + ".new", 3)
    with open(os.path.join(rolling + ".new", STATE_FILE), "w") as f:
        f.write('{"next_ep')
    os.rename(rolling, rolling + ".old")
    _recover_rolling(rolling)
    assert epoch_of(rolling) == 2
    # A rolling checkpoint whose loop state does not parse gives way to a complete retired one.
    shutil.rmtree(rolling + ".old", ignore_errors=True)
    shutil.copytree(rolling, rolling + ".old")
    with open(os.path.join(rolling, STATE_FILE), "w") as f:
        f.write("")
    _recover_rolling(rolling)
    assert epoch_of(rolling) == 2 and not os.path.exists(rolling + ".old")


def test_safetensors_write_replaces_the_file_whole(tmp_path):
    """Written beside the target and moved over it (SafetensorsWriter.cs:46-58): no .tmp remains and the
    file reads back."""
    from laya_amd.safetensors_io import SafetensorsFile, write
    path = str(tmp_path / "t.safetensors")
    write(path, [("a", (2, 3), np.arange(6, dtype=np.float32), "F32")])
    write(path, [("b", (4,), np.ones(4, np.float32), "BF16")])
    assert not os.path.exists(path + ".tmp")
    st = SafetensorsFile(path)
    assert list(st.entries) == ["b"]
    np.testing.assert_array_equal(st.read_float32("b"), np.ones(4, np.float32))
