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


def _valid(ks, skv):
    return ks if 0 <= ks <= skv else 0


def _sim_rows(kernel, kstart, B, Hq, Sq, Skv, D, causal):
    """The forward's / pass 1's loops, transcribed: per (head, 128-row block) the key tiles from the
    diagonal one down to the recorded first processed key, per wavefront unless wholly above its rows."""
    bn = 64 if kernel == "coalibi_fwd_kernel" else 32
    KS, DT = D // 16, max(D, 32) // 32
    per = 2 * KS + (4 if bn == 64 else 2) * DT
    nqb, n = (Sq + 127) // 128, 0
    for bh in range(B * Hq):
        for qb in range(nqb):
            q0 = qb * 128
            last = min(q0 + 127, Skv - 1) if causal else Skv - 1
            nkt = last // bn + 1
            kt0 = _valid(int(kstart[bh][qb]), Skv) // bn
            for kt in range(nkt - 1, kt0 - 1, -1):
                for w in range(4):
                    if causal and kt * bn > q0 + 32 * w + 31:
                        continue
                    n += per
    return n


def _sim_pass2(kernel, kstart, B, Hq, Hkv, Sq, Skv, D, causal):
    """Pass 2's work list, transcribed: per key head and 64-key block, per query head of the group,
    the 64-row tiles from the last one whose row block processed the block down to the first that
    can see it; per wavefront (key group, query half) when that half holds a processed visible pair."""
    KS, DT = D // 16, max(D, 32) // 32
    per = 4 * DT + (2 * KS if kernel == "coalibi_bwd_dkdv_kernel" else 0)
    g = Hq // Hkv
    nqt, nrb, nkb, n = (Sq + 63) // 64, (Sq + 127) // 128, (Skv + 63) // 64, 0
    for b in range(B):
        for hkv in range(Hkv):
            for kb in range(nkb):
                kwg0 = kb * 64
                qt0 = min(kwg0 // 64, nqt) if causal else 0
                for gi in range(g):
                    ks = kstart[b * Hq + hkv * g + gi]
                    hi = qt0 - 1
                    for rb in range(nrb):
                        if _valid(int(ks[rb]), Skv) <= kwg0:
                            hi = max(hi, min(2 * rb + 1, nqt - 1))
                    for qt in range(hi, qt0 - 1, -1):
                        processed = _valid(int(ks[qt // 2]), Skv) <= kwg0
                        for kg in range(2):
                            for qh in range(2):
                                kw0, qs0 = kwg0 + 32 * kg, qt * 64 + 32 * qh
                                if processed and kw0 < Skv and qs0 < Sq and (not causal or qs0 + 31 >= kw0):
                                    n += per
    return n


def test_issued_products_match_the_kernel_loops():
    """profiling.issued_k16 (vectorised) against the kernels' loops transcribed one by one, for
    random recorded first keys (multiples of 64, and out-of-range values that the kernels read as
    0), causal and not, square and rectangular, grouped heads; and the full-work forward at the
    headline shape: every 64-key x 32-row tile at or below the diagonal."""
    import numpy as np

    rng = np.random.default_rng(7)
    for (B, Hq, Hkv, Sq, Skv, D, causal) in [(1, 4, 2, 300, 300, 64, True), (2, 2, 2, 500, 260, 128, True),
                                             (1, 3, 3, 200, 700, 32, False), (1, 2, 1, 1000, 1000, 16, True)]:
        nqb = (Sq + 127) // 128
        ks = rng.integers(0, (Skv + 63) // 64, size=(B * Hq, nqb)) * 64
        ks[0, 0] = Skv + 5   # out of range: read as 0
        ks[-1, -1] = -64
        for kern in ("coalibi_fwd_kernel", "coalibi_bwd_dq_kernel"):
            want = _sim_rows(kern, ks, B, Hq, Sq, Skv, D, causal)
            assert profiling.issued_k16(kern, ks, B, Hq, Hkv, Sq, Skv, D, causal) == want, kern
        for kern in ("coalibi_bwd_dkdv_store_kernel", "coalibi_bwd_dkdv_kernel"):
            want = _sim_pass2(kern, ks, B, Hq, Hkv, Sq, Skv, D, causal)
            assert profiling.issued_k16(kern, ks, B, Hq, Hkv, Sq, Skv, D, causal) == want, kern
    # headline, nothing skipped: per (head, 128-row block qb), wavefront w processes tiles 0 ..
    # (128 qb + 32 w + 31) // 64, each 2*8 + 4*4 = 32 products
    zero = np.zeros((64, 32), dtype=np.int64)
    per_head = sum(((128 * qb + 32 * w + 31) // 64 + 1) for qb in range(32) for w in range(4))
    assert profiling.issued_k16("coalibi_fwd_kernel", zero, 4, 16, 16, 4096, 4096, 128) == 64 * per_head * 32
    # ... which is the algorithmic causal forward plus the diagonal tiles' masked halves
    fwd, _ = profiling.attention_flops(4, 16, 4096, 4096, 128)
    issued = 64 * per_head * 32 * profiling.K16_FLOPS
    assert 1.0 < issued / fwd < 1.03
