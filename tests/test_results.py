"""The results pipeline's report (lowbit_amd/results.py) on a synthetic result: the
reference's row schema (src/lowbit/bench.py:209-227) plus the GPU fields, and the
tables of src/lowbit/report.py:44-101 with the reference's published rows beside."""
from lowbit_amd import results as R

REF_FIELDS = {"phase", "M", "N", "K", "threads", "cache", "method", "format", "isa", "params", "reps",
              "t_median_s", "t_min_s", "gflops", "weight_bytes", "weight_gbps", "speedup_vs_numpy_fp32",
              "max_rel_err"}


def _row(m, n, k, fmt, cache, t, layout):
    wb = n * k // 2 + n * (k // 128) * 4
    roof, frac = R._roofline(fmt, layout, m, n, k, t, wb)
    return {"phase": "decode" if m == 1 else "batch", "M": m, "N": n, "K": k, "threads": None, "cache": cache,
            "method": f"{fmt} gfx950", "format": fmt, "isa": "gfx950", "params": None, "reps": 7,
            "t_median_s": t, "t_min_s": t * 0.98, "gflops": 2.0 * m * n * k / t / 1e9, "weight_bytes": wb,
            "weight_gbps": wb / t / 1e9, "speedup_vs_numpy_fp32": None, "max_rel_err": 2e-7,
            "device": "gfx950", "weight_layout": layout, "roofline": roof, "roofline_frac": frac}


def test_report_tables_and_schema():
    rows = [_row(1, 11008, 4096, f, c, 7.6e-6, "row-major") for f in R.FORMATS for c in ("hot", "cold")]
    rows += [_row(64, 11008, 4096, f, "hot", 20e-6, "t16") for f in R.FORMATS]
    res = {"meta": {"date": "2026-12-01", "device": "gfx950 (256 CUs)", "timing": "graph"}, "rows": rows}
    for r in rows:
        assert REF_FIELDS <= set(r)
    md = R.report(res)
    assert "Decode, M=1, N=11008, K=4096" in md and "cold cache" in md
    # the reference's best 4-thread W4A8 cold row (621 us) and its speedup sit beside the GPU row
    assert "w4a8 avx512-vnni | 621.0 µs | 38.6 | 82×" in md
    assert "| 64 | 11008 | 4096 |" in md and "2164.8" in md
    frac = R._roofline("w4a8", "t16", 64, 11008, 4096, 20e-6, 0)[1]
    assert abs(frac - 2 * 64 * 11008 * 4096 / 20e-6 / 5e15) < 1e-12


def test_reference_table_covers_the_published_shapes():
    for (m, n, k) in R.DECODE_SHAPES:
        for f in R.FORMATS:
            assert (m, n, k, f, "cold") in R.REFERENCE_4T and (m, n, k, f, "hot") in R.REFERENCE_4T
    for (m, n, k) in R.BATCH_SHAPES[:4]:
        for f in R.FORMATS:
            assert (m, n, k, f, "hot") in R.REFERENCE_4T


def test_report_group32_table():
    rows = [_row(1, 11008, 4096, f, "cold", 7.6e-6, "row-major") for f in R.FORMATS]
    r = _row(1, 11008, 4096, "w4a8", "cold", 8.0e-6, "row-major")
    r.update(format="w4a8-g32", method="w4a8-g32 gfx950")
    rows.append(r)
    md = R.report({"meta": {"date": "d", "device": "gfx950", "timing": "graph"}, "rows": rows})
    assert "groups of 32" in md and "| 1 | 11008 | 4096 | cold | w4a8-g32 gfx950 |" in md
