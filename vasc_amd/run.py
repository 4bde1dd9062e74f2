"""Run launcher: local JSON settings, the dataset evaluator's command line,
its launch record, and the evaluator process itself.

``python -m vasc_amd.run [--config PATH] [overrides]`` runs one evaluation of
a backbone (VGGT or Pi3) in one attention mode (dense, topk, vasc) with the
release switches of ``vasc_amd.launcher.method_environment`` and the
per-layer sparsity profile. ``--dry-run`` prints the launch record instead;
``--init-config`` copies ``vasc_amd/configs/local.example.json`` to
``configs/local.json`` (never overwriting).

Behaviour follows the reference launcher (``evaluate.py:83-296``): the same
options and defaults, the same config keys and validation, the same
evaluator options and ``launch.json`` fields. The code is organised
differently:

* ``SETTINGS`` is one table of every setting (type, default, choices, help);
  the command-line parser and the validation of the JSON file are both
  derived from it.
* ``EVALUATORS`` describes each backbone's evaluator (script, checkout
  option, dense flag, extra flags, point budget per dataset, checkouts it
  needs); ``plan_launch`` turns resolved settings into a ``LaunchPlan``
  (command, environment, record, required paths) without touching the
  filesystem.
* ``execute`` is the only part with side effects: dependency checks, the
  output folder, ``launch.json``, the evaluator process with its output
  streamed to ``run.log``, and the ``metrics.json`` check.

The evaluator runs this build: its ``PYTHONPATH`` starts with
``vasc_amd/compat`` (a ``sparse_vggt`` import shim whose modules are
``vasc_amd``'s) and the runtime root. The dataset evaluators themselves live
under ``--evaluation-root`` (not part of this build).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import subprocess
import sys
from dataclasses import dataclass, field
from datetime import datetime
from pathlib import Path

from .launcher import CONFIG, MODES, allocation_settings, layer_sparsity_string, method_environment

ROOT = Path(__file__).resolve().parents[1]
EXAMPLE = Path(__file__).resolve().parent / "configs" / "local.example.json"
SHIM = Path("vasc_amd") / "compat"  # relative to the runtime root


# ------------------------------------------------------------------ settings
@dataclass(frozen=True)
class Setting:
    """One run setting: its JSON key (also the option's dest), its kind, and
    the command line's default, choices and help. ``needed`` settings must
    come from the config file or the command line. A path default is
    relative to the repository root."""
    key: str
    kind: str  # "choice", "path", "text", "int", "float", "bool", "switch"
    default: object = None
    choices: tuple = ()
    needed: bool = False
    help: str | None = None

    @property
    def flag(self) -> str:
        return "--" + self.key.replace("_", "-")


SETTINGS = (
    Setting("backbone", "choice", choices=("vggt", "pi3"), needed=True),
    Setting("mode", "choice", "vasc", choices=MODES),
    Setting("dataset", "choice", choices=("7scenes", "nrgbd"), needed=True),
    Setting("data_root", "path", needed=True),
    Setting("weights", "path", needed=True),
    Setting("vggt_root", "path", "external/vggt"),
    Setting("pi3_root", "path", "external/Pi3"),
    Setting("streamvggt_root", "path", "external/StreamVGGT"),
    Setting("runtime_root", "path", ".", help="Directory holding the vasc_amd package"),
    Setting("evaluation_root", "path", "evaluation", help="Directory holding the dataset evaluators"),
    Setting("output", "path", help="Exact output directory; otherwise create a timestamped run"),
    Setting("output_root", "path", "outputs", help="Parent directory for automatic runs"),
    Setting("gpu", "text", "0"),
    Setting("sparsity", "float", 0.75),
    Setting("structural_allocation", "switch", None,
            help="Enable/disable the fixed cross-layer budget profile above 70%% sparsity (enabled by default)"),
    Setting("stride", "int", CONFIG["stride"]),
    Setting("scene", "text"),
    Setting("sequence", "text"),
    Setting("frame_limit", "int", help="Explicit short test; omitted for paper evaluation"),
    Setting("warmup", "int", 0),
    Setting("repeats", "int", 1),
    Setting("pose_only", "switch", False),
)
BY_KEY = {s.key: s for s in SETTINGS}


def _root() -> Path:
    # looked up at call time: tests point the launcher at a scratch repository
    return ROOT


def _resolve(value) -> Path:
    """A path setting: ``~`` expanded, relative paths taken from the repository root."""
    path = Path(value).expanduser()
    return (path if path.is_absolute() else _root() / path).resolve()


def _well_typed(setting: Setting, value) -> bool:
    """Whether a JSON value suits the setting (booleans are not numbers here)."""
    if setting.kind in ("path", "text", "choice"):
        return isinstance(value, str) and bool(value.strip())
    if setting.kind == "switch":
        return type(value) is bool
    if setting.kind == "int":
        return type(value) is int
    return type(value) in (int, float)


def load_run_config(path) -> dict:
    """The settings of a local JSON file, checked against ``SETTINGS``:
    every key known, every value of its setting's type and (for choices)
    among its choices; paths resolved. Raises ValueError."""
    try:
        data = json.loads(Path(path).read_text(encoding="utf-8-sig"))
    except json.JSONDecodeError as exc:
        raise ValueError(f"malformed JSON: {exc}") from None
    if not isinstance(data, dict):
        raise ValueError("run config must be a JSON object")
    strangers = sorted(k for k in data if k not in BY_KEY)
    if strangers:
        raise ValueError("unknown config key(s): " + ", ".join(strangers))
    settings = {}
    for key, value in data.items():
        setting = BY_KEY[key]
        if not _well_typed(setting, value):
            raise ValueError(f"invalid type or empty value for config key: {key}")
        if setting.choices and value not in setting.choices:
            raise ValueError(f"invalid {key}: {value}; choose from {', '.join(setting.choices)}")
        settings[key] = _resolve(value) if setting.kind == "path" else value
    return settings


def parser(defaults: dict | None = None) -> argparse.ArgumentParser:
    """The command line, one option per setting; ``defaults`` (the local
    config) fill in values and make needed settings optional."""
    defaults = dict(defaults or {})
    cli = argparse.ArgumentParser(
        description=__doc__.splitlines()[0],
        usage="%(prog)s [--config PATH] [overrides]\n       %(prog)s --init-config [--config PATH]",
        epilog="Configure paths once in configs/local.json; CLI overrides are optional.")
    cli.add_argument("--config", type=Path, help="Local JSON settings; defaults to configs/local.json when present")
    cli.add_argument("--init-config", action="store_true",
                     help="Create local settings from the example without overwriting an existing file")
    converters = {"path": Path, "text": str, "int": int, "float": float, "choice": str}
    budget = None
    for s in SETTINGS:
        default = _root() / s.default if s.kind == "path" and s.default is not None else s.default
        if s.key == "structural_allocation":
            # the switch and its older spelling --allocation exclude each other
            budget = cli.add_mutually_exclusive_group()
            budget.add_argument(s.flag, action=argparse.BooleanOptionalAction, default=default, help=s.help)
            budget.add_argument("--allocation", choices=("paper", "uniform"), default=None,
                                help="Compatibility alias: paper enables structural allocation, uniform disables it")
            continue
        if s.kind == "switch":
            cli.add_argument(s.flag, action=argparse.BooleanOptionalAction, default=default, help=s.help)
            continue
        cli.add_argument(s.flag, type=converters[s.kind], default=default, help=s.help,
                         choices=s.choices or None, required=s.needed and s.key not in defaults)
    cli.add_argument("--dry-run", action="store_true")
    cli.set_defaults(**defaults)
    return cli


def run_allocation(args) -> dict:
    """The structural-allocation record of the parsed options
    (``launcher.allocation_settings``): ``--allocation`` when given, then the
    ``--[no-]structural-allocation`` switch, then the configured default."""
    if args.allocation is not None:
        enabled = args.allocation == "paper"
    else:
        enabled = args.structural_allocation
    return allocation_settings(args.backbone, args.mode, args.sparsity, enabled)


# ---------------------------------------------------------------- evaluators
@dataclass(frozen=True)
class Evaluator:
    """How one backbone's dataset evaluator is called."""
    script: str
    checkout: str                 # the setting naming the upstream model checkout
    dense_flag: str               # flag that runs the unmodified model
    flags: tuple = ()             # always passed
    point_budget: dict = field(default_factory=dict)  # dataset -> --max_points
    needs: tuple = ()             # (setting, sub-path) pairs that must exist for a real run


EVALUATORS = {
    "vggt": Evaluator("eval_7scenes_sparse_vggt.py", "vggt_root", "--vanilla_vggt", ("--aux_output",),
                      {"nrgbd": 999999}, (("vggt_root", "vggt"),)),
    "pi3": Evaluator("eval_pi3_sparse.py", "pi3_root", "--dense", (), {"7scenes": 200000, "nrgbd": 200000},
                     (("vggt_root", "vggt"), ("pi3_root", "pi3"))),
}

# option checks of a launch: (violated?, message)
RULES = (
    (lambda a: a.stride < 1 or a.warmup < 0 or a.repeats < 1,
     "stride/repeats must be positive and warmup nonnegative"),
    (lambda a: a.frame_limit is not None and a.frame_limit < 1, "frame-limit must be positive"),
    (lambda a: bool(a.sequence) and (a.dataset != "7scenes" or not a.scene), "sequence requires a 7scenes scene"),
    (lambda a: a.dataset == "7scenes" and bool(a.scene) and not a.sequence,
     "a single 7scenes scene requires --sequence"),
    (lambda a: not math.isfinite(a.sparsity), "sparsity must be a finite number"),
)


@dataclass
class LaunchPlan:
    """Everything a run needs, computed without side effects."""
    command: list
    environment: dict
    output: Path
    allocation: dict
    frame_policy: str
    required: list

    def record(self, config: Path | None) -> dict:
        """The launch record (``launch.json``, and the dry run's output)."""
        shown = ("HIP_VISIBLE_DEVICES", "CUDA_VISIBLE_DEVICES", "PYTHONPATH")
        rec = {
            "command": self.command,
            "environment": {k: v for k, v in self.environment.items() if k.startswith("SPARSE_VGGT_") or k in shown},
            "frame_policy": self.frame_policy,
            "allocation": self.allocation,
        }
        if config is not None and config.is_file():
            rec["config"] = {"path": str(config), "sha256": hashlib.sha256(config.read_bytes()).hexdigest()}
        return rec


def _output_dir(args, allocation: dict) -> Path:
    if args.output is not None:
        return Path(args.output).resolve()
    stamp = datetime.now().strftime("%Y%m%d-%H%M%S-%f")
    tag = f"{args.backbone}_{args.dataset}_{args.mode}_s{args.sparsity:g}_{allocation['effective_policy']}"
    return (Path(args.output_root) / f"{tag}_{stamp}").resolve()


def plan_launch(args) -> LaunchPlan:
    """The evaluator command, environment and record of parsed options.
    Raises ValueError on inconsistent options (including a sparsity outside
    [0, 1) or a profile that would leave it)."""
    for violated, message in RULES:
        if violated(args):
            raise ValueError(message)
    allocation = run_allocation(args)
    spec = EVALUATORS[args.backbone]
    out = _output_dir(args, allocation)
    options = [
        ("weights", Path(args.weights).resolve()),
        ("dataset", args.dataset),
        ("data_root", Path(args.data_root).resolve()),
        (spec.checkout, Path(getattr(args, spec.checkout)).resolve()),
        ("streamvggt_root", Path(args.streamvggt_root).resolve()),
        ("output_dir", out / "reconstruction"),
        ("metrics_json", out / "metrics.json"),
        ("kf_every", args.stride),
        ("timing_warmup", args.warmup),
        ("timing_repeats", args.repeats),
        ("max_points", spec.point_budget.get(args.dataset)),
        ("scene", args.scene or None),
        ("seq_id", args.sequence or None),
        ("num_frames", args.frame_limit or None),
    ]
    flags = list(spec.flags)
    if args.mode == "dense":
        flags.append(spec.dense_flag)
    else:
        options += [("sparse_ratio", args.sparsity), ("cdf_threshold", "none")]
        if allocation["applied"]:
            # the profile's own %.10f text, which the evaluators parse back
            options.append(("layer_sparsity", layer_sparsity_string(args.backbone, args.sparsity, "paper")))
    if args.pose_only:
        flags.append("--pose_only")
    command = [sys.executable, str(Path(args.evaluation_root) / spec.script), *flags]
    for name, value in options:
        if value is not None:
            command += ["--" + name, str(value)]

    runtime = Path(args.runtime_root).resolve()
    search = [runtime / SHIM, runtime, Path(args.pi3_root).resolve(), Path(args.vggt_root).resolve()]
    env = {k: v for k, v in os.environ.items() if not k.startswith("SPARSE_VGGT_") and k != "PYTHONPATH"}
    env.update(method_environment(args.backbone, args.mode))
    env.update(HIP_VISIBLE_DEVICES=args.gpu, CUDA_VISIBLE_DEVICES=args.gpu, PYTHONUNBUFFERED="1",
               PYTHONPATH=os.pathsep.join(str(p) for p in search))

    required = [Path(args.weights), Path(args.data_root), Path(args.streamvggt_root) / "src/eval/mv_recon",
                Path(command[1])]
    required += [Path(getattr(args, key)) / sub for key, sub in spec.needs]
    required += [runtime / "vasc_amd", runtime / SHIM / "sparse_vggt"]
    policy = "full_sequence_after_stride" if args.frame_limit is None else "explicit_limit"
    return LaunchPlan(command, env, out, allocation, policy, required)


def build_launch(args):
    """``(command, environment)`` of parsed options (see ``plan_launch``)."""
    plan = plan_launch(args)
    return plan.command, plan.environment


# ------------------------------------------------------------------- running
class LaunchError(Exception):
    """A launch that cannot start (missing inputs, occupied output folder)."""


def _preflight(plan: LaunchPlan, backbone: str) -> None:
    for path in plan.required:
        if not path.exists():
            raise LaunchError(f"missing dependency: {path}; check configs/local.json")
    if backbone == "pi3":
        # eval_pi3_sparse.py:251 imports the reconstruction protocol, which this build does not ship
        raise LaunchError("the Pi3 evaluator needs sparse_vggt.evaluation.pi3_reconstruction (the reference's "
                          "reconstruction protocol), which is not part of this build; use --dry-run for the command")
    if plan.output.exists() and (not plan.output.is_dir() or any(plan.output.iterdir())):
        raise LaunchError("output path is not an empty directory; choose a new output directory")


def execute(plan: LaunchPlan, record: dict, backbone: str, mode: str, gpu: str) -> Path:
    """Run the evaluator of ``plan``; returns the metrics file. Raises
    LaunchError before starting anything, SystemExit when the evaluator fails."""
    _preflight(plan, backbone)
    plan.output.mkdir(parents=True, exist_ok=True)
    (plan.output / "launch.json").write_text(json.dumps(record, indent=2), encoding="utf-8")
    log_path = plan.output / "run.log"
    print(f"Running {backbone}/{mode} on GPU {gpu}; log: {log_path}", flush=True)
    with log_path.open("w", encoding="utf-8") as log, subprocess.Popen(
            plan.command, env=plan.environment, cwd=_root(), stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
            text=True, encoding="utf-8", errors="replace", bufsize=1) as child:
        for line in child.stdout:
            for sink in (log, sys.stdout):
                sink.write(line)
                sink.flush()
        status = child.wait()
    if status:
        raise SystemExit(f"Evaluation failed ({status}); see {log_path}")
    metrics = plan.output / "metrics.json"
    if not metrics.is_file():
        raise SystemExit("Evaluator did not produce metrics.json")
    return metrics


def _init_config(dest: Path, explicit: bool, fail) -> None:
    try:
        dest.parent.mkdir(parents=True, exist_ok=True)
        with dest.open("x", encoding="utf-8") as handle:
            handle.write(EXAMPLE.read_text(encoding="utf-8"))
    except OSError as exc:
        fail(f"cannot create config (existing files are never overwritten): {exc}")
    hint = "python -m vasc_amd.run" + (f' --config "{dest}"' if explicit else "")
    print(f"Created {dest}. Set weights and data_root, then run {hint}.")


def main(argv=None) -> None:
    argv = list(sys.argv[1:] if argv is None else argv)
    if {"-h", "--help"} & set(argv):
        parser().parse_args(argv)
    front = argparse.ArgumentParser(add_help=False)
    front.add_argument("--config", type=Path)
    front.add_argument("--init-config", action="store_true")
    known, others = front.parse_known_args(argv)
    config = (known.config or _root() / "configs" / "local.json").expanduser().resolve()
    if known.init_config:
        if others:
            front.error("--init-config only accepts --config to choose the destination")
        _init_config(config, known.config is not None, front.error)
        return
    defaults = {}
    if known.config is not None or config.exists():
        try:
            defaults = load_run_config(config)
        except (OSError, ValueError) as exc:
            front.error(f"cannot load {config}: {exc}")
    if not argv and not defaults:
        front.error("no local config; start with python -m vasc_amd.run --init-config")
    cli = parser(defaults)
    args = cli.parse_args(argv)
    try:
        plan = plan_launch(args)
    except ValueError as exc:
        cli.error(str(exc))
    record = plan.record(config)
    if args.dry_run:
        print(json.dumps(record, indent=2))
        return
    try:
        metrics = execute(plan, record, args.backbone, args.mode, args.gpu)
    except LaunchError as exc:
        cli.error(str(exc))
    print(f"Results: {metrics.resolve()}")


if __name__ == "__main__":
    main()
