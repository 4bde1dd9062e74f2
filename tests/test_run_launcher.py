"""The run launcher (vasc_amd.run) against the behaviour the reference's own
launcher tests pin (tests/test_release.py:18-163, tests/test_run_config.py:
17-184): the release matrix of commands and switches, the structural
allocation interfaces, dry-run records, environment isolation, local JSON
settings and their validation, init-config, automatic output folders and a
real launch of a stand-in evaluator with its log and launch record. CPU only.
"""
import hashlib
import io
import json
import os
from contextlib import redirect_stderr, redirect_stdout
from pathlib import Path
from unittest.mock import patch

import pytest

from vasc_amd import launcher, run

EXAMPLE = json.loads(run.EXAMPLE.read_text())


def _args(*extra):
    return run.parser().parse_args(["--backbone", "vggt", "--dataset", "nrgbd", "--weights", "model.pt",
                                    "--data-root", "data/nrgbd", "--output", "outputs/test", *extra])


def _opt(cmd, name):
    return cmd[cmd.index(name) + 1]


# ------------------------------------------------------------- release matrix
def test_main_matrix():
    for model in ("vggt", "pi3"):
        for mode in launcher.MODES:
            for sparsity in launcher.CONFIG["sparsities"]:
                args = _args("--backbone", model, "--mode", mode, "--sparsity", str(sparsity))
                cmd, env = run.build_launch(args)
                assert _opt(cmd, "--kf_every") == "10"
                assert "--num_frames" not in cmd
                assert env["SPARSE_VGGT_QK_PV_THRESHOLD"] == "1e10"
                assert ("--layer_sparsity" in cmd) == (mode != "dense" and sparsity > .70)
                assert run.run_allocation(args)["enabled"]
                assert _opt(cmd, "--max_points") == ("200000" if model == "pi3" else "999999")
                assert cmd[1].endswith("eval_7scenes_sparse_vggt.py" if model == "vggt" else "eval_pi3_sparse.py")
                assert ("--vanilla_vggt" in cmd or "--dense" in cmd) == (mode == "dense")


def test_structural_switch_matrix():
    for model in ("vggt", "pi3"):
        for mode in launcher.MODES:
            for sparsity in launcher.CONFIG["sparsities"]:
                for enabled in (False, True):
                    base = ("--backbone", model, "--mode", mode, "--sparsity", str(sparsity))
                    flag = "--structural-allocation" if enabled else "--no-structural-allocation"
                    args = _args(*base, flag)
                    legacy = _args(*base, "--allocation", "paper" if enabled else "uniform")
                    assert run.build_launch(args) == run.build_launch(legacy)
                    s = run.run_allocation(args)
                    assert s["enabled"] == enabled
                    assert s["applied"] == (enabled and mode != "dense" and sparsity > .70)
                    ratios = s["layer_sparsities"]
                    assert len(ratios) == launcher.CONFIG["structural"][model]["layers"]
                    assert sum(ratios) / len(ratios) == pytest.approx(0 if mode == "dense" else sparsity, abs=1e-9)
                    if not s["applied"]:
                        assert len(set(ratios)) == 1


def test_layer_profile_text_round_trips():
    cmd, _ = run.build_launch(_args("--sparsity", "0.75"))
    values = [float(v) for v in _opt(cmd, "--layer_sparsity").split(",")]
    assert values == launcher.layer_sparsity("vggt", 0.75) and len(values) == 24
    assert values[11] == pytest.approx(0.70) and values[0] == pytest.approx(0.7666666667)


def test_allocation_changes_only_layer_schedule():
    for model in ("vggt", "pi3"):
        for mode in launcher.MODES:
            base = ("--backbone", model, "--mode", mode)
            on, on_env = run.build_launch(_args(*base, "--structural-allocation"))
            off, off_env = run.build_launch(_args(*base, "--no-structural-allocation"))
            assert on_env == off_env
            if "--layer_sparsity" in on:
                i = on.index("--layer_sparsity")
                del on[i:i + 2]
            assert on == off


def test_allocation_config_default_and_override():
    for default in (False, True):
        with patch.dict(launcher.CONFIG["structural"], {"enabled": default}):
            s = run.run_allocation(_args())
            assert s["enabled"] == default and s["applied"] == default
            for flags, enabled in ((("--structural-allocation",), True), (("--no-structural-allocation",), False),
                                   (("--allocation", "paper"), True), (("--allocation", "uniform"), False)):
                assert run.run_allocation(_args(*flags))["enabled"] == enabled


def test_allocation_cli_conflicts():
    for flag in ("--structural-allocation", "--no-structural-allocation"):
        for legacy in ("paper", "uniform"):
            for argv in ((flag, "--allocation", legacy), ("--allocation", legacy, flag)):
                with redirect_stderr(io.StringIO()), pytest.raises(SystemExit):
                    _args(*argv)


def test_allocation_threshold_and_extreme_sparsity():
    for model in ("vggt", "pi3"):
        for sparsity in (0, .70, .7001, .85):
            args = _args("--backbone", model, "--sparsity", str(sparsity), "--structural-allocation")
            assert run.run_allocation(args)["applied"] == (sparsity > .70)
        with pytest.raises(ValueError):  # the profile would leave [0, 1)
            run.build_launch(_args("--backbone", model, "--sparsity", ".99", "--structural-allocation"))
        for extra in (("--no-structural-allocation",), ("--mode", "dense", "--structural-allocation")):
            command, _ = run.build_launch(_args("--backbone", model, "--sparsity", ".99", *extra))
            assert "--layer_sparsity" not in command


def test_dry_run_records_allocation():
    for extra, policy in ((("--structural-allocation",), "paper"), (("--no-structural-allocation",), "uniform"),
                          (("--structural-allocation", "--mode", "dense"), "dense"),
                          (("--structural-allocation", "--sparsity", ".65"), "uniform")):
        args = _args("--dry-run", *extra)
        out = io.StringIO()
        with patch.object(run, "parser") as parser_mock, redirect_stdout(out):
            parser_mock.return_value.parse_args.return_value = args
            run.main(["--dry-run"])
        record = json.loads(out.getvalue())
        assert record["allocation"] == run.run_allocation(args)
        assert record["allocation"]["effective_policy"] == policy
        command = record["command"]
        if record["allocation"]["applied"]:
            assert [float(v) for v in _opt(command, "--layer_sparsity").split(",")] == \
                record["allocation"]["layer_sparsities"]
        else:
            assert "--layer_sparsity" not in command


def test_environment_isolation_and_gpu_selection():
    with patch.dict(os.environ, {"SPARSE_VGGT_BAD_EXPERIMENT": "1", "PYTHONPATH": "old"}):
        _, env = run.build_launch(_args("--gpu", "3"))
    assert "SPARSE_VGGT_BAD_EXPERIMENT" not in env
    assert env["PYTHONPATH"] != "old" and str(run.ROOT) in env["PYTHONPATH"].split(os.pathsep)
    assert env["HIP_VISIBLE_DEVICES"] == env["CUDA_VISIBLE_DEVICES"] == "3"
    assert {k: v for k, v in env.items() if k.startswith("SPARSE_VGGT_")} == launcher.method_environment("vggt", "vasc")


def test_supported_modes():
    assert launcher.MODES == ("dense", "topk", "vasc")
    assert launcher.method_environment("vggt", "vasc")["SPARSE_VGGT_COSA_VALUE_RISK_PAIR_DEBT"] == "1"
    for mode in ("current", "memory"):
        with pytest.raises(ValueError):
            launcher.method_environment("vggt", mode)
        with redirect_stderr(io.StringIO()), pytest.raises(SystemExit):
            _args("--mode", mode)


@pytest.mark.parametrize("extra", [("--stride", "0"), ("--sparsity", "nan"), ("--sparsity", "1"),
                                   ("--sequence", "seq-01"), ("--frame-limit", "0")])
def test_bad_inputs(extra):
    with pytest.raises(ValueError):
        run.build_launch(_args(*extra))


def test_seven_scenes_scene_and_sequence():
    base = ("--dataset", "7scenes")
    with pytest.raises(ValueError):
        run.build_launch(_args(*base, "--scene", "chess"))
    cmd, _ = run.build_launch(_args(*base, "--scene", "chess", "--sequence", "seq-03", "--frame-limit", "5"))
    assert _opt(cmd, "--scene") == "chess" and _opt(cmd, "--seq_id") == "seq-03" and _opt(cmd, "--num_frames") == "5"
    assert "--max_points" not in cmd  # VGGT on 7-Scenes keeps the evaluator's default


# ------------------------------------------------------------- local settings
@pytest.fixture
def cfg(tmp_path):
    path = tmp_path / "run.json"

    def write(data=None):
        path.write_text(json.dumps(EXAMPLE if data is None else data), encoding="utf-8")
        return path

    def dry(*extra):
        out = io.StringIO()
        with redirect_stdout(out):
            run.main(["--config", str(path), "--dry-run", *extra])
        return json.loads(out.getvalue())

    return tmp_path, path, write, dry


def test_config_paths_are_repository_relative(cfg):
    _, path, write, _ = cfg
    write()
    d = run.load_run_config(path)
    assert d["weights"] == run.ROOT / "checkpoints/vggt/model.pt"
    assert d["data_root"] == run.ROOT / "data/nrgbd"
    assert d["structural_allocation"] is True and d["gpu"] == "0"


def test_cli_overrides_config(cfg):
    root, _, write, dry = cfg
    write()
    record = dry("--mode", "topk", "--sparsity", ".65", "--gpu", "2", "--no-structural-allocation",
                 "--output", str(root / "custom"))
    assert record["allocation"]["requested_sparsity"] == .65 and not record["allocation"]["enabled"]
    assert record["environment"]["CUDA_VISIBLE_DEVICES"] == "2"
    assert record["environment"]["SPARSE_VGGT_COSA_VALUE_RISK_PAIR_DEBT"] == "0"
    assert str(root / "custom" / "metrics.json") in record["command"]
    assert not (root / "custom").exists()


def test_both_allocation_interfaces_override_config(cfg):
    _, _, write, dry = cfg
    for initial in (False, True):
        write({**EXAMPLE, "structural_allocation": initial})
        for flags, expected in ((("--structural-allocation",), True), (("--no-structural-allocation",), False),
                                (("--allocation", "paper"), True), (("--allocation", "uniform"), False)):
            assert dry(*flags)["allocation"]["enabled"] == expected


def test_structural_default_and_opt_out(cfg):
    _, _, write, dry = cfg
    for value in (None, False, True):
        data = dict(EXAMPLE)
        if value is None:
            data.pop("structural_allocation")
        else:
            data["structural_allocation"] = value
        write(data)
        s = dry()["allocation"]
        assert s["enabled"] == (value is not False) and s["applied"] == (value is not False)


def test_auto_output_and_provenance(cfg):
    root, path, write, dry = cfg
    write({**EXAMPLE, "output_root": str(root / "outputs")})
    first, second = dry(), dry()
    assert first["command"] != second["command"]  # timestamped run folders
    metrics = Path(_opt(first["command"], "--metrics_json"))
    assert metrics.parent.parent == root / "outputs"
    assert "vggt_nrgbd_vasc_s0.75_paper_" in metrics.parent.name
    assert not (root / "outputs").exists()
    assert first["config"]["sha256"] == hashlib.sha256(path.read_bytes()).hexdigest()


def test_pose_only_can_be_disabled_from_cli(cfg):
    _, _, write, dry = cfg
    write({**EXAMPLE, "pose_only": True})
    assert "--pose_only" in dry()["command"]
    assert "--pose_only" not in dry("--no-pose-only")["command"]


@pytest.mark.parametrize("key,value", [("structural_allocation", "false"), ("gpu", 0), ("weights", ""),
                                       ("weights", None), ("frame_limit", 2.5), ("stride", True),
                                       ("pose_only", "yes"), ("mode", "unknown"), ("mode", "current"),
                                       ("mode", "memory"), ("sparsity", True), ("sparisty", .75),
                                       ("allocation", "paper")])
def test_bad_config_values(cfg, key, value):
    _, path, write, _ = cfg
    write({**EXAMPLE, key: value})
    with pytest.raises(ValueError):
        run.load_run_config(path)


@pytest.mark.parametrize("text", ["[]", "null", "{broken"])
def test_non_object_and_malformed_json(cfg, text):
    _, path, _, _ = cfg
    path.write_text(text)
    with pytest.raises(ValueError):
        run.load_run_config(path)


def test_missing_explicit_config_fails(cfg):
    _, _, _, dry = cfg
    with redirect_stderr(io.StringIO()), pytest.raises(SystemExit):
        dry()


def test_init_never_overwrites_and_rejects_run_flags(cfg):
    root, path, _, _ = cfg
    with redirect_stdout(io.StringIO()):
        run.main(["--init-config", "--config", str(path)])
    before = path.read_bytes()
    assert json.loads(before) == EXAMPLE
    with redirect_stderr(io.StringIO()), pytest.raises(SystemExit):
        run.main(["--init-config", "--config", str(path)])
    assert path.read_bytes() == before
    other = root / "other.json"
    with redirect_stderr(io.StringIO()), pytest.raises(SystemExit):
        run.main(["--init-config", "--config", str(other), "--mode", "dense"])
    assert not other.exists()


def test_default_local_config_and_setup_message(tmp_path):
    out = io.StringIO()
    with patch.object(run, "ROOT", tmp_path), redirect_stderr(out), pytest.raises(SystemExit):
        run.main([])
    assert "--init-config" in out.getvalue()
    config = tmp_path / "configs" / "local.json"
    config.parent.mkdir()
    config.write_text(json.dumps(EXAMPLE))
    out = io.StringIO()
    with patch.object(run, "ROOT", tmp_path), redirect_stdout(out):
        run.main(["--dry-run"])
    record = json.loads(out.getvalue())
    assert Path(record["config"]["path"]) == config.resolve()
    assert str(tmp_path / "checkpoints/vggt/model.pt") in record["command"]


def test_plain_launch_with_a_stand_in_evaluator_and_no_overwrite(tmp_path):
    """The real subprocess, log and launch-record path with a stand-in
    evaluator that writes metrics.json; a second launch into the same
    (now non-empty) output folder is refused and changes nothing."""
    config = tmp_path / "configs/local.json"
    config.parent.mkdir()
    config.write_text(json.dumps({**EXAMPLE, "output": "outputs/result", "runtime_root": str(run.ROOT)}))
    (tmp_path / "checkpoints/vggt").mkdir(parents=True)
    (tmp_path / "checkpoints/vggt/model.pt").touch()
    for folder in ("data/nrgbd", "external/StreamVGGT/src/eval/mv_recon", "external/vggt/vggt", "evaluation"):
        (tmp_path / folder).mkdir(parents=True)
    # the stand-in imports what the reference's evaluator imports (eval_7scenes_sparse_vggt.py:939-941,
    # 1115-1118) and records which files those names resolve to
    (tmp_path / "evaluation/eval_7scenes_sparse_vggt.py").write_text(
        "import json, os, pathlib, sys\n"
        "import sparse_vggt\n"
        "from sparse_vggt.utils import sparse_wrapper\n"
        "from sparse_vggt.models.vggt import sparse_aggregator_from_vggt\n"
        "from sparse_vggt.models.vggt_layerwise import sparse_aggregator_from_vggt_layerwise\n"
        "import vasc_amd.install, vasc_amd.sparse_wrapper\n"
        "path = pathlib.Path(sys.argv[sys.argv.index('--metrics_json') + 1])\n"
        "path.write_text(json.dumps({'stand_in': True, 'mode': os.environ['SPARSE_VGGT_COSA_VALUE_RISK_PAIR_DEBT'],\n"
        "    'wrapper': sparse_wrapper.__file__,\n"
        "    'same_wrapper': sparse_wrapper is vasc_amd.sparse_wrapper,\n"
        "    'same_installers': sparse_aggregator_from_vggt is vasc_amd.install.sparse_aggregator_from_vggt\n"
        "        and sparse_aggregator_from_vggt_layerwise is vasc_amd.install.sparse_aggregator_from_vggt_layerwise}))\n"
        "print('stand-in evaluation finished')\n", encoding="utf-8")
    with patch.object(run, "ROOT", tmp_path), redirect_stdout(io.StringIO()):
        run.main(["--evaluation-root", str(tmp_path / "evaluation")])
    out = tmp_path / "outputs/result"
    metrics = json.loads((out / "metrics.json").read_text())
    assert metrics == {"stand_in": True, "mode": "1", "wrapper": str(run.ROOT / "vasc_amd" / "sparse_wrapper.py"),
                       "same_wrapper": True, "same_installers": True}
    assert "stand-in evaluation finished" in (out / "run.log").read_text()
    launch = json.loads((out / "launch.json").read_text())
    assert launch["allocation"]["applied"]
    snapshot = {p.name: p.read_bytes() for p in out.iterdir()}
    with patch.object(run, "ROOT", tmp_path), redirect_stderr(io.StringIO()), pytest.raises(SystemExit):
        run.main(["--evaluation-root", str(tmp_path / "evaluation")])
    assert {p.name: p.read_bytes() for p in out.iterdir()} == snapshot


def test_pi3_launch_is_refused_before_anything_runs(tmp_path):
    """The Pi3 evaluator imports the reconstruction protocol this build does
    not ship (eval_pi3_sparse.py:251): a real launch stops with that reason
    and leaves no output folder; its dry run still prints the command."""
    config = tmp_path / "configs/local.json"
    config.parent.mkdir()
    config.write_text(json.dumps({**EXAMPLE, "backbone": "pi3", "output": "outputs/pi3",
                                  "runtime_root": str(run.ROOT)}))
    (tmp_path / "checkpoints/vggt").mkdir(parents=True)
    (tmp_path / "checkpoints/vggt/model.pt").touch()
    for folder in ("data/nrgbd", "external/StreamVGGT/src/eval/mv_recon", "external/vggt/vggt", "external/Pi3/pi3",
                   "evaluation"):
        (tmp_path / folder).mkdir(parents=True)
    (tmp_path / "evaluation/eval_pi3_sparse.py").write_text("raise SystemExit(3)\n")
    err = io.StringIO()
    with patch.object(run, "ROOT", tmp_path), redirect_stderr(err), pytest.raises(SystemExit):
        run.main(["--evaluation-root", str(tmp_path / "evaluation")])
    assert "pi3_reconstruction" in err.getvalue()
    assert not (tmp_path / "outputs/pi3").exists()
    out = io.StringIO()
    with patch.object(run, "ROOT", tmp_path), redirect_stdout(out):
        run.main(["--evaluation-root", str(tmp_path / "evaluation"), "--dry-run"])
    record = json.loads(out.getvalue())
    assert record["command"][1].endswith("eval_pi3_sparse.py") and _opt(record["command"], "--max_points") == "200000"
    assert record["environment"]["PYTHONPATH"].split(os.pathsep)[0] == str(run.ROOT / "vasc_amd" / "compat")


def test_settings_table_drives_parser_and_config():
    """Every setting is both a config key and a command-line option, with
    the same default the parser reports."""
    cli = run.parser({"backbone": "vggt", "dataset": "nrgbd", "weights": Path("w"), "data_root": Path("d")})
    ns = cli.parse_args([])
    for s in run.SETTINGS:
        assert hasattr(ns, s.key)
        if s.kind == "path" and s.default is not None:
            assert getattr(ns, s.key) == run.ROOT / s.default
        elif s.key not in ("backbone", "dataset", "weights", "data_root"):
            assert getattr(ns, s.key) == s.default
    assert {s.key for s in run.SETTINGS} == set(json.loads(run.EXAMPLE.read_text())) | {
        "runtime_root", "evaluation_root", "output", "output_root", "stride", "scene", "sequence", "frame_limit",
        "warmup", "repeats", "pose_only"}
