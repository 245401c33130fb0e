"""The rocprofv3 summaries of co_alibi_attn/profiling.py on synthetic CSV input: the traffic
calibration and the counter normalisation (no GPU, no profiler)."""
import csv
import os

from co_alibi_attn import profiling

FWD = "void coalibi::(anonymous namespace)::coalibi_fwd_kernel<_Float16, 128, true>(coalibi::FwdArgs)"
COPY = "__amd_rocclr_copyBuffer"


def write_pmc(directory, rows):
    os.makedirs(directory, exist_ok=True)
    with open(os.path.join(directory, "pmc_counter_collection.csv"), "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Process_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for pid, did, name, counter, value in rows:
            w.writerow(dict(Process_Id=pid, Dispatch_Id=did, Kernel_Name=name, Counter_Name=counter,
                            Counter_Value=value))


def test_traffic_is_scaled_by_the_calibration_copy(tmp_path):
    gib_kib = profiling.CALIBRATION_BYTES / 1024
    # FETCH_SIZE reads half the copied bytes for the copy (factor 2); WRITE_SIZE reads all (factor 1).
    # Instances of one dispatch are summed: two rows of 100 KiB make 200 KiB.
    write_pmc(tmp_path / "f", [(1, 1, COPY, "FETCH_SIZE", gib_kib / 2), (1, 2, FWD, "FETCH_SIZE", 100.0),
                               (1, 2, FWD, "FETCH_SIZE", 100.0), (1, 3, FWD, "FETCH_SIZE", 300.0)])
    write_pmc(tmp_path / "w", [(1, 1, COPY, "WRITE_SIZE", gib_kib), (1, 2, FWD, "WRITE_SIZE", 50.0),
                               (1, 3, FWD, "WRITE_SIZE", 150.0)])
    out = tmp_path / "traffic.md"
    profiling.main(["traffic", str(tmp_path / "f"), str(tmp_path / "w"), "--command", "x", "--out", str(out)])
    got = profiling.read_traffic(str(out))
    # mean fetch 250 KiB x 2 + mean write 100 KiB x 1
    assert abs(got["coalibi_fwd_kernel"] - (250 * 2 + 100) * 1024) < 1


def test_counter_normalisation(tmp_path):
    T = 1000.0  # active cycles per XCD
    simds = 4 * profiling.MI355X_CUS
    a = [(1, 1, FWD, "GRBM_GUI_ACTIVE", profiling.MI355X_XCDS * T), (1, 1, FWD, "SQ_INSTS_MFMA", 100.0),
         (1, 1, FWD, "SQ_INSTS_VALU", 1200.0), (1, 1, FWD, "SQ_INSTS_VALU_TRANS_F32", 300.0),
         (1, 1, FWD, "SQ_INSTS_LDS", 50.0)]
    b = [(1, 1, FWD, "GRBM_GUI_ACTIVE", profiling.MI355X_XCDS * T),
         (1, 1, FWD, "SQ_VALU_MFMA_BUSY_CYCLES", 0.25 * simds * T),
         (1, 1, FWD, "SQ_ACTIVE_INST_VALU", 0.5 * simds * T / 4), (1, 1, FWD, "SQ_ACTIVE_INST_LDS", 100.0),
         (1, 1, FWD, "SQ_LDS_BANK_CONFLICT", 80.0)]
    write_pmc(tmp_path / "a", a)
    write_pmc(tmp_path / "b", b)
    stats = tmp_path / "stats.md"
    stats.write_text("| kernel | calls | average (us) | min (us) | max (us) | share |\n|---|\n"
                     "| `coalibi_fwd_kernel` | 2 | 500.0 | 1 | 1 | 1 % |\n")
    traffic = tmp_path / "traffic.md"
    traffic.write_text("    traffic_bytes_per_launch coalibi_fwd_kernel 1000000000\n")
    out = tmp_path / "counters.md"
    profiling.main(["counters", str(tmp_path / "a"), str(tmp_path / "b"), "--command", "x", "--traffic",
                    str(traffic), "--stats", str(stats), "--out", str(out)])
    row = [line for line in out.read_text().splitlines() if line.startswith("| `coalibi_fwd_kernel`")][0]
    cells = [c.strip() for c in row.split("|")[1:-1]]
    # MFMA busy, VALU busy, VALU/MFMA, trans/MFMA, LDS/MFMA, conflict per LDS instr, conflict share, GB/s
    assert cells[1:] == ["25.0 %", "50.0 %", "12.00", "3.00", "0.50", "1.600", "20.0 %", "2000"]


def test_attention_flops_closed_form():
    """FlashAttention convention: fwd 4*B*Hq*Sq*Skv*D, halved when causal, bwd 2.5x.  At the
    headline shape that is 2.749e11 / 6.872e11 flops; the reference's own harness counts the
    full square with bwd 2x (benchmark_flops.py:139-140), i.e. 2x the causal forward here."""
    from co_alibi_attn.profiling import attention_flops

    fwd, bwd = attention_flops(4, 16, 4096, 4096, 128, causal=True)
    assert fwd == 4 * 4 * 16 * 4096 * 4096 * 128 / 2 and round(fwd / 1e11, 3) == 2.749
    assert bwd == 2.5 * fwd and round(bwd / 1e11, 3) == 6.872
    ref_fwd = 4 * 4 * 16 * 4096 * 4096 * 128  # benchmark_flops.py:139
    assert ref_fwd == 2 * fwd
    nc_fwd, nc_bwd = attention_flops(1, 2, 100, 300, 64, causal=False)
    assert nc_fwd == 4 * 2 * 100 * 300 * 64 and nc_bwd == 2.5 * nc_fwd
    # one product of the per-kernel accounting is half the forward
    assert attention_flops(1, 1, 8, 8, 32, causal=True)[0] == 2 * (2 * 32 * 8 * 8 / 2)
