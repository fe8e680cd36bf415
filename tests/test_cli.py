"""The command line: the reference's CLI contract (tests/test_cli_smoke.py of
the reference: parser fields, dry-run lines, target validation, choices) and
this build's calibrate command; GPU runs of demo --fused and calibrate."""

import pytest

from decodebench_amd.cli import SWEEP_HEADER, build_parser, main


def test_cli_parser_demo():
    args = build_parser().parse_args(["demo", "f1", "--dim", "2048", "--batch", "4", "--dry-run"])
    assert (args.command, args.name, args.dim, args.batch, args.dry_run) == \
        ("demo", "f1", 2048, 4, True)
    assert args.fused is False


def test_cli_parser_profile():
    args = build_parser().parse_args(["profile", "module.py:build_fn", "--trials", "50",
                                      "--dry-run"])
    assert (args.command, args.target, args.trials, args.dry_run) == \
        ("profile", "module.py:build_fn", 50, True)


def test_cli_parser_sweep():
    args = build_parser().parse_args(["sweep", "f4", "--batch", "1,2,4", "--dim", "2048",
                                      "--dry-run"])
    assert (args.command, args.name, args.batch, args.dim, args.dry_run) == \
        ("sweep", "f4", [1, 2, 4], 2048, True)


def test_cli_dry_run_outputs(capsys):
    assert main(["demo", "f1", "--dim", "4096", "--batch", "1", "--dry-run"]) == 0
    assert "[dry-run] demo f1 with dim=4096, batch=1" in capsys.readouterr()[0]
    assert main(["profile", "user_module.py:build_seq", "--dry-run"]) == 0
    assert "[dry-run] profile target user_module.py:build_seq" in capsys.readouterr()[0]
    assert main(["sweep", "f2", "--batch", "1,2", "--dim", "4096", "--dry-run"]) == 0
    assert "[dry-run] sweep demo f2 with batch=[1, 2], dim=4096" in capsys.readouterr()[0]
    assert main(["demo", "f4", "--fused", "--dry-run"]) == 0
    assert "fused=hip" in capsys.readouterr()[0]


def test_cli_profile_validation(capsys):
    assert main(["profile", "user_module.py"]) == 2
    err = capsys.readouterr()[1]
    assert "Error: Target must be in the format 'path/to/module.py:build_fn'" in err
    assert main(["profile", "/nonexistent/m.py:build"]) == 1
    assert "does not exist" in capsys.readouterr()[1]


def test_cli_invalid_choices():
    with pytest.raises(SystemExit):
        build_parser().parse_args(["demo", "invalid_name"])
    with pytest.raises(SystemExit):
        build_parser().parse_args(["sweep", "f1", "--batch", "1,x"])


def test_cli_calibrate_validation(capsys):
    assert main(["calibrate"]) == 2
    assert "--null" in capsys.readouterr()[1]
    assert main(["calibrate", "--null", "--iters", "0"]) == 2
    assert main(["calibrate", "--null", "--gate-g2", "--dry-run"]) == 0
    assert "[dry-run] calibrate null gate-g2" in capsys.readouterr()[0]
    assert main(["calibrate", "--vendor-f4", "--kv-len", "0"]) == 2
    assert main(["calibrate", "--vendor-f4", "--kv-len", "1024", "--dry-run"]) == 0
    assert "vendor-f4 with iters=default, rotate=True, kv_len=1024, kv_batch=1" in \
        capsys.readouterr()[0]


def test_sweep_csv_header_matches_the_reference():
    assert SWEEP_HEADER == ["demo", "dim", "batch", "trials", "t_stream_us", "t_graph_us",
                            "delta_launch_us", "b_bytes_est_us", "bound", "total_bytes",
                            "eliminable_bytes", "ci_lo", "ci_hi"]


@pytest.mark.gpu
def test_cli_calibrate_on_gpu(capsys):
    assert main(["calibrate", "--null", "--gate-g2", "--iters", "40"]) == 0
    out = capsys.readouterr()[0]
    for line in ("t_launch_stream:", "t_launch_graph:", "t_kernel_in_graph:",
                 "GEMV d_out=14336 d_in=4096", "Ratio (ours/"):
        assert line in out
    assert "G2: PASS" in out or "G2: FAIL" in out


@pytest.mark.gpu
def test_cli_calibrate_vendor_f4(capsys):
    # F4 against torch SDPA at L=1024: also an independent check of F4's output.
    assert main(["calibrate", "--vendor-f4", "--kv-len", "1024", "--kv-batch", "2"]) == 0
    out = capsys.readouterr()[0]
    for line in ("F4 attention B=2 Hq=32 Hkv=8 D=128 L=1024", "Ours (db_f4_splitkv):",
                 "torch SDPA:", "max |ours - SDPA|:"):
        assert line in out


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["f1", "f2", "f4"])
def test_cli_demo_with_fused_kernel(name, tmp_path, capsys):
    csv_path = tmp_path / "trials.csv"
    assert main(["demo", name, "--dim", "2048", "--trials", "3", "--fused",
                 "--csv", str(csv_path)]) == 0
    out = capsys.readouterr()[0]
    assert "Measured fused latency" in out
    assert csv_path.exists() and "fused" in csv_path.read_text()
