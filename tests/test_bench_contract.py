"""bench.py's command-line contract on the CPU: more than one GPU is refused
with a message before anything touches a device."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, cwd=REPO)


def test_more_than_one_gpu_is_refused():
    for n in ("2", "8"):
        r = _bench("--gpus", n, "--steps", "1", "--warmup", "0")
        assert r.returncode == 2, r.stderr
        assert r.stdout == ""                      # no JSON line
        assert "one GPU only" in r.stderr


def test_help_lists_the_driver_flags():
    r = _bench("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup"):
        assert flag in r.stdout


def test_summary_is_last_and_fits_the_kept_tail():
    """The compact per-configuration summary must fit in the 2,000 characters
    of output a driver keeps, and name every configuration."""
    import json

    import bench

    ro = {"avg_launch_us": 14.4, "frac": 0.61, "rocprof_avg_us": 14.5, "rocprof_frac": 0.6}
    kern = {f"fp8_e4m3_gemv {n}x{k} T={t}": {"us": 3.0, "frac_of_peak": 0.2, "kernel_over_floor": 1.3}
            for n, k in ((1536, 4096), (576, 4096), (4096, 4096), (4096, 2048)) for t in (1, 8)}
    kern.update({f"fp8_e4m3_gemv {nm} {n}x{k} T={t}": {"us": 9.0, "frac_of_peak": 0.5, "kernel_over_floor": 1.2}
                 for nm, n, k in (("wq_b", 32768, 1024), ("wo_b", 4096, 8192)) for t in (1, 8)})
    kern.update({f"rmsnorm_fuse_residual_add T={t}x4096": {"us": 2.7, "frac_of_peak": 0.01} for t in (1, 8, 64)})
    kern["mxfp4_gemv_m1 2048x4096"] = {"us": 3.1, "frac_of_peak": 0.18, "kernel_over_floor": 1.4}
    cfg = {"cfg3_T4": {"moe_layer_us": 81.6, "hbm_frac_of_peak": 0.63},
           "cfg3_T16": {"moe_layer_us": 241.4, "hbm_frac_of_peak": 0.71},
           "routed_dispatch_T1": {"us": 23.9, "hbm_frac_of_peak": 0.43},
           "cfg4_decode": {"us_per_layer": 23.7, "hbm_frac_of_peak": 0.56},
           "cfg4_prefill": {"us_per_layer": 797.4, "hbm_frac_of_peak": 0.53, "mfma_frac_of_bf16_peak": 0.1,
                            "read_floor": {"layer_bytes": {"kernel_over_floor": 1.5}}}}
    r = {"config": {"tokens": 1}, "moe_layer_us": 23.6, "hbm_frac_of_peak": 0.57, "roofline": ro,
         "stage_b_roofline": ro, "configs": cfg, "kernels": kern,
         "read_floor": {"layer_one_pass": {"kernel_over_floor": 1.39}},
         "cpu_baseline": {"us_per_layer": 2.1e6, "cores": 16}}
    s = bench.summary(r)
    for k in ("cfg3_T1", "cfg3_T4", "cfg3_T16", "dispatch_T1", "cfg4_decode_layer", "cfg4_prefill_layer",
              "stageA", "stageB", "cfg0_mxfp4", "fp8_576x4096_T8", "fp8_4096x8192_T8", "cfg1_rmsnorm_T64",
              "cpu_baseline"):
        assert k in s, k
    assert len(json.dumps(s, separators=(",", ":"))) < 1700


def test_profile_lines_go_stale_with_their_sources(tmp_path, monkeypatch):
    """A TRAFFIC / DURATION line of profiles/*.md is used only while the
    kernel sources it names hash as the profile's SOURCE lines record."""
    import bench

    prof = tmp_path / "profiles"
    prof.mkdir()
    sha = bench.source_sha("rmsnorm_fuse.hip")
    (prof / "p.md").write_text(
        f"SOURCE rmsnorm_fuse.hip {sha}\nSOURCE fp8_e4m3_gemv.hip 000000000000\n"
        "TRAFFIC rms@T1 4096 rmsnorm_fuse.hip\nTRAFFIC fp8@T1 8192 fp8_e4m3_gemv.hip\n"
        "DURATION rms@T1 2.5 100 rmsnorm_fuse.hip\nTRAFFIC nosrc@T1 1 missing.hip\n")
    monkeypatch.setattr(bench, "REPO", str(tmp_path))
    assert bench.profiled_traffic("rms@T1") == (4096, "profiles/p.md")
    assert bench.profiled_duration("rms@T1") == (2.5, "profiles/p.md")
    assert bench.profiled_traffic("fp8@T1") == (None, None)      # source changed since the profile
    assert bench.profiled_traffic("nosrc@T1") == (None, None)
