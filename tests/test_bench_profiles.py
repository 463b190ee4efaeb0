"""The committed profiles carry, for each benchmark configuration, the two
figures bench.py reads beside its own stage timing: the HBM traffic of one
launch of the dominant kernel (rocprofv3 --pmc) and that kernel's average
duration in the kernel trace (rocprofv3 --kernel-trace).  CPU only."""

import bench


def test_every_config_has_traffic_and_trace_lines():
    for cfg in range(5):
        traffic, src = bench.traffic_from_profile("w13", cfg)
        assert traffic is not None and traffic > 0, cfg
        us, tsrc = bench.trace_from_profile("w13", cfg)
        assert us is not None and us > 0, cfg
        assert src == tsrc, (cfg, src, tsrc)


def test_trace_roofline_uses_the_same_definition():
    # 417,595,392 algorithmic bytes per w13 launch at M=16 (118 touched
    # experts x 3,538,944 B) over the trace average is the trace frac
    us, _ = bench.trace_from_profile("w13", 1)
    frac = 417_595_392 / (us * 1e-6) / (bench.HBM_PEAK_GBS * 1e9)
    assert 0.5 < frac < 0.8


def test_unknown_kernel_has_no_profile_line():
    assert bench.trace_from_profile("w2", 1) == (None, None)
    assert bench.traffic_from_profile("w13", 9) == (None, None)
