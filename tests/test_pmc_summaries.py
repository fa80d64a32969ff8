"""The rocprofv3 counter summaries (zhip.pmc) on hand-made CSVs (CPU only).

The committed HBM-traffic and matrix-core summaries are computed by these functions from rocprofv3's
counter_collection.csv / kernel_trace.csv; here they read small files whose answers are known.
"""
import csv
import json
import os

from zhip import pmc

COLS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def write_csv(path, rows, cols=COLS):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=cols)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(cols, r)))


def test_traffic_summary_scales_by_the_copy(tmp_path):
    copy = pmc.COPY_BYTES
    # the copy reads 1.25x its bytes in FETCH_SIZE KiB and 1.0x in WRITE_SIZE; the kernel 2 x 1000 KiB read
    # (split over two counter instances), 10 KiB written
    fetch = [("1", "__amd_rocclr_copyBuffer", "FETCH_SIZE", copy / 1024 * 1.25)]
    write = [("1", "__amd_rocclr_copyBuffer", "WRITE_SIZE", copy / 1024)]
    for d in range(2, 5):
        fetch += [(str(d), "void zh::mv_kernel<12, 12, 1, 2, 64, 1>(zh::MvParams)", "FETCH_SIZE", 500.0)] * 2
        write += [(str(d), "void zh::mv_kernel<12, 12, 1, 2, 64, 1>(zh::MvParams)", "WRITE_SIZE", 10.0)]
    write_csv(str(tmp_path / "fetch" / "x" / "pmc_counter_collection.csv"), fetch)
    write_csv(str(tmp_path / "write" / "x" / "pmc_counter_collection.csv"), write)
    meta = {"position": 4096, "kernels": {"gate_up": {"us": 1.0, "algorithmic": {"mv_kernel<12, 12, 1, 2, 64": 819200}}}}
    json.dump(meta, open(tmp_path / "meta.json", "w"))
    out = tmp_path / "s.md"
    pmc.main(["summarize", str(tmp_path / "fetch"), str(tmp_path / "write"), str(tmp_path / "meta.json"),
              "--out", str(out)])
    want = int(round(1000 * 1024 / 1.25 + 10 * 1024))  # 819200 + 10240
    assert pmc.read_traffic(str(out)) == want
    assert "| 1.0125 |" in out.read_text()


def test_mfma_summary_groups_shapes_and_prices_flops(tmp_path):
    cols = COLS + ["Start_Timestamp", "End_Timestamp"]
    rows = []
    # a shape of 2^20 MOPS (0.537 GFLOP) in 1 us, busy 512 of 1000 GUI cycles per SIMD
    for d in (1, 2):
        for name, v in (("SQ_INSTS_VALU_MFMA_MOPS_F16", 1 << 20), ("SQ_VALU_MFMA_BUSY_CYCLES", 512 * 1024),
                        ("GRBM_GUI_ACTIVE", 1000)):
            rows.append((str(d), "void zh::qgemm_kernel<8, 0, true, 2>(zh::QGemmParams)", name, v, 0, 1000))
    # a kernel with no matrix-core work is left out
    rows.append(("3", "void zh::mv_kernel<8, 8, 0, 1, 64, 1>(zh::MvParams)", "SQ_INSTS_VALU_MFMA_MOPS_F16", 0, 0, 500))
    write_csv(str(tmp_path / "m" / "x" / "pmc_counter_collection.csv"), rows, cols)
    out = tmp_path / "m.md"
    pmc.main(["mfma", str(tmp_path / "m"), "--title", "t", "--command", "c", "--out", str(out)])
    text = out.read_text()
    tf = (1 << 20) * 512 / 1000 / 1e3
    assert f"| 2 | {(1 << 20) * 512 / 1e9:.3f} | 1.00 | {tf:.1f} |" in text
    assert "| 51.20 |" in text
    assert "mv_kernel" not in text


def test_request_size_summary_counts_bytes_by_size(tmp_path):
    rows = []
    # the calibration copy (the largest copyBuffer dispatch) reads 128-byte requests only; a small upload
    # copy must not be taken for it
    for did, name, vals in ((1, "__amd_rocclr_copyBuffer", (0, 0, pmc.COPY_BYTES // 128, pmc.COPY_BYTES // 128)),
                            (2, "__amd_rocclr_copyBuffer", (0, 3, 1, 4)),
                            (3, "void zh::attn_mfma_kernel<128, 4, false>(zh::AttnParams)", (10, 1000, 500, 1510))):
        for c, v in zip(pmc.REQ_COUNTERS, vals):
            rows.append((str(did), name, c, v))
    write_csv(str(tmp_path / "r" / "x" / "pmc_counter_collection.csv"), rows)
    meta = {"position": 4096, "kernels": {"attention": {"us": 1.0, "algorithmic": {"attn_mfma_kernel<128": 128320}}}}
    json.dump(meta, open(tmp_path / "meta.json", "w"))
    out = tmp_path / "r.md"
    pmc.main(["reqsize", str(tmp_path / "r"), str(tmp_path / "meta.json"), "--out", str(out)])
    text = out.read_text()
    assert "1.0000 of the copy" in text
    assert "| 128320 | 128320 | 1.0000 |" in text  # 10 x 32 + 1000 x 64 + 500 x 128
