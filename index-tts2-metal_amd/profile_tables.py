"""Builds the summaries under profiles/ from raw rocprofv3 output (measurement tooling).

One command rebuilds every table from the CSVs a profiling run leaves in a
directory RAW (the commands below write there):

    python3 index-tts2-metal_amd/profile_tables.py --raw RAW [--out profiles]

It reads whichever of these inputs exist and writes the summary each one feeds:

  trace/bench_kernel_trace.csv, trace/bench_kernel_stats.csv, trace.log, bench_plain.log
      rocprofv3 --kernel-trace --stats -T --output-format csv -d RAW/trace -o bench --
          python3 -u bench.py --no-cpu-baseline --no-cpu-1thread --gpt-codes 0      (trace.log)
      python3 -u bench.py --no-cpu-baseline --no-cpu-1thread --gpt-codes 0          (bench_plain.log)
    -> cfm_decode_T860_S25_B2_kernel_trace.md   stats, per-op table of the T=860 decodes
       cfm_decode_configs_kernel_trace.md       per-op tables of every other decode shape
                                                 (T=128 12 steps, T=3000 25 steps, the padded
                                                 8-request batch with and without skipped padding)
       condition_producer_codes350_kernel_trace.md, bigvgan_T860_kernel_trace.md
  pmc_{sq,mem,l2,fetch,write}/p_counter_collection.csv
      rocprofv3 --pmc <pass counters> --output-format csv -d RAW/pmc_<pass> -o p --
          python3 -u index-tts2-metal_amd/profile_kernels.py --launches 20
    -> decode_kernels_T860_counters.md
  pmc_bfetch/fetch_counter_collection.csv, pmc_bwrite/write_counter_collection.csv, pmc_bench.log
      rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) -T --output-format csv -d RAW/pmc_bfetch -o fetch --
          python3 -u bench.py <short run, see BENCH_PMC>
    -> traffic_gemm_wavenet_conv_gate_T860.json
  gpttrace/bench_kernel_trace.csv, gpttrace/bench_kernel_stats.csv, gpt_trace.log,
  gptpmc_fetch/fetch_counter_collection.csv, gptpmc_write/write_counter_collection.csv
      the same with MIT2CFM_GRAPH=0 and the GPT section of bench.py (see GPT_CMDS)
    -> gpt_decode_P150_553codes_kernel_trace.md, traffic_gemv_gpt_c_fc.json

Any of these CSVs may come gzip-compressed (NAME.csv.gz); it is unpacked first.

HBM bytes come from FETCH_SIZE and WRITE_SIZE (KiB per dispatch) scaled by what the
same counters read for the bench's 256 MiB streaming copy (`calibration` in the bench
line): FETCH_SIZE reads half the bytes a copy fetches on MI355X, so its factor is
about 2,048 bytes per KiB; WRITE_SIZE's is 1,024.
"""
from __future__ import annotations

import argparse
import collections
import csv
import gzip
import json
import shutil
from pathlib import Path

PEAK_TF = 2500.0  # MI355X f16 dense MFMA, TFLOP/s
TRACE_CMD = ("rocprofv3 --kernel-trace --stats -T --output-format csv -d $RAW/trace -o bench -- "
             "python3 -u bench.py --no-cpu-baseline --no-cpu-1thread --gpt-codes 0")
PLAIN_CMD = "python3 -u bench.py --no-cpu-baseline --no-cpu-1thread --gpt-codes 0 > $RAW/bench_plain.log"
PMC_PASSES = {
    "sq": "SQ_WAVES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_WAIT_INST_ANY SQ_INSTS_VMEM SQ_INST_LEVEL_VMEM "
          "SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 GRBM_GUI_ACTIVE GRBM_COUNT",
    "mem": "TA_BUSY_avr TA_ADDR_STALLED_BY_TC_CYCLES_sum TD_TD_BUSY_sum TD_TC_STALL_sum TCP_TCC_READ_REQ_sum "
           "TCP_TCC_READ_REQ_LATENCY_sum TCP_PENDING_STALL_CYCLES_sum TCP_UTCL1_TRANSLATION_MISS_sum GRBM_GUI_ACTIVE",
    "l2": "TCC_HIT_sum TCC_MISS_sum TCC_EA0_RDREQ_sum TCC_TAG_STALL_sum SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT "
          "SQ_WAIT_INST_LDS SQ_INST_LEVEL_LDS SQ_INSTS_SALU SQ_INSTS_VALU GRBM_GUI_ACTIVE",
    "fetch": "FETCH_SIZE",
    "write": "WRITE_SIZE",
}
PMC_PROG = "python3 -u index-tts2-metal_amd/profile_kernels.py --launches 20"
BENCH_PMC = ("python3 -u bench.py --steps 1 --warmup 1 --no-cpu-baseline --no-cpu-1thread --no-configs "
             "--kernel-launches 5 --voc-calls 0 --acoustic-calls 0 --cond-calls 1 --gpt-codes 0")
GPT_BENCH = ("python3 -u bench.py --steps 1 --warmup 1 --no-cpu-baseline --no-configs --kernel-launches 5 "
             "--voc-calls 0 --acoustic-calls 0 --cond-calls 1")
GPT_CMDS = [
    f"MIT2CFM_GRAPH=0 rocprofv3 --kernel-trace --stats -T --output-format csv -d $RAW/gpttrace -o bench -- {GPT_BENCH}",
    f"MIT2CFM_GRAPH=0 rocprofv3 --pmc FETCH_SIZE -T --output-format csv -d $RAW/gptpmc_fetch -o fetch -- {GPT_BENCH}",
    f"MIT2CFM_GRAPH=0 rocprofv3 --pmc WRITE_SIZE -T --output-format csv -d $RAW/gptpmc_write -o write -- {GPT_BENCH}",
]


# ---------------------------------------------------------------------------- inputs
def load_trace(path: Path) -> list[dict]:
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return rows


def dur(r: dict) -> float:
    """Kernel duration in microseconds."""
    return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0


def bench_line(path: Path) -> dict | None:
    if not path.exists():
        return None
    lines = [x for x in open(path) if x.startswith("{")]
    return json.loads(lines[-1]) if lines else None


def md_table(header: list[str], rows: list[list]) -> str:
    out = ["| " + " | ".join(header) + " |", "|" + "---|" * len(header)]
    out += ["| " + " | ".join(str(c) for c in r) + " |" for r in rows]
    return "\n".join(out)


# ---------------------------------------------------------------------------- decodes
# One Euler step of the decode graph, 86 dispatches (engine.hip enqueue_decode):
# the per-step merge, 13 blocks (QKV, attention, wo, w1|w3, then w2 -- or for
# blocks 6..11 w2 folded with the next block's skip-in), the final AdaRMSNorm,
# the post GEMM, 8 WaveNet layers (k=5 conv + gate, res/skip; the last one's
# res/skip has N=512 and adds res_projection), the final AdaLN and the folded
# final linear + conv2 + CFG + Euler update.  A decode is 4 set-up dispatches
# (prep, key bias, the two step-invariant merge GEMMs), S steps and a copy.
STEP_ORDER = ["merge"]
for _l in range(13):
    STEP_ORDER += ["qkv", "attn", "wo", "w13", "fold" if 6 <= _l <= 11 else "w2"]
STEP_ORDER += ["adarms", "post"]
for _l in range(8):
    STEP_ORDER += ["conv", "resskip" if _l < 7 else "finalskip"]
STEP_ORDER += ["adaln", "conv2_euler"]
assert len(STEP_ORDER) == 86
KERNEL_OF = {"attn": "attention_kernel", "adarms": "adarms_kernel", "adaln": "adaln_kernel",
             "conv2_euler": "conv2_euler_kernel"}


def op_flops(op: str, B: int, T: int) -> float:
    """Algorithmic FLOPs of one launch at B branches of T rows (model K, not padded K)."""
    R = B * T
    mnk = {"merge": (512, 80), "qkv": (1536, 512), "wo": (512, 512), "w13": (3072, 512), "w2": (512, 1536),
           "fold": (512, 2560), "post": (1024, 592), "conv": (1024, 2560), "resskip": (1024, 512),
           "finalskip": (512, 512)}
    if op in mnk:
        n, k = mnk[op]
        return 2.0 * R * n * k
    if op == "attn":
        return 2048.0 * B * T * T  # QK^T and PV: 2 x 2 x 64 FLOP per (query, key, head), 8 heads
    return 0.0


def find_decodes(rows: list[dict]):
    """(B, T, S, segment) for every whole decode in the trace."""
    out = []
    for i, r in enumerate(rows):
        if "decode_prep_kernel" not in r["Kernel_Name"]:
            continue
        T, B = int(r["Grid_Size_X"]) // 256, int(r["Grid_Size_Y"])
        j = i + 1
        while j < len(rows) and "copy_f32_kernel" not in rows[j]["Kernel_Name"] and j - i < 200000:
            j += 1
        if j >= len(rows):
            continue
        n = j - i + 1
        if (n - 5) % 86:
            continue
        S = (n - 5) // 86
        seg = rows[i:j + 1]
        ok = True
        for s in range(S):
            for k, op in enumerate(STEP_ORDER):
                name = seg[4 + s * 86 + k]["Kernel_Name"]
                want = KERNEL_OF.get(op, "gemm_kernel")
                # long sequences run the QKV product in its row-resident kernel
                ok = ok and (want in name or (op == "qkv" and "qkv_rows_kernel" in name))
        if ok:
            out.append((B, T, S, seg))
    return out


def skipped_padding_flops(tokens: list[int], T: int) -> dict:
    """Algorithmic FLOPs per launch of each op when padded rows are skipped:
    every product covers min(valid + 2, T) rows of each of a request's two
    branches, the attention those rows' queries against the valid keys."""
    need = [min(t + 2, T) for t in tokens for _ in range(2)]
    keys = [t for t in tokens for _ in range(2)]
    out = {op: op_flops(op, 1, 1) * sum(need) for op in STEP_ORDER if op != "attn" and op_flops(op, 1, 1)}
    out["attn"] = 2048.0 * sum(n * k for n, k in zip(need, keys))
    return out


def decode_table(group: list, B: int, T: int, S: int, flops: dict | None = None) -> tuple[str, dict]:
    per = collections.defaultdict(list)
    spans, busy = [], []
    for seg in group:
        spans.append((int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])) / 1000.0)
        busy.append(sum(dur(r) for r in seg))
        for s in range(S):
            for k, op in enumerate(STEP_ORDER):
                per[op].append(dur(seg[4 + s * 86 + k]))
    cnt = collections.Counter(STEP_ORDER)
    tot = {op: sum(v) / len(v) * cnt[op] for op, v in per.items()}
    step = sum(tot.values())
    rows = []
    summary = {}
    for op in sorted(tot, key=lambda o: -tot[o]):
        avg = tot[op] / cnt[op]
        fl = flops[op] if flops and op in flops else op_flops(op, B, T)
        tf = fl / (avg * 1e-6) / 1e12 if fl else None
        summary[op] = (avg, tf / PEAK_TF if tf else None)
        rows.append([f"`{op}`", cnt[op], f"{tot[op]:.1f}", f"{avg:.2f}", f"{100 * tot[op] / step:.1f}%",
                     f"{tf:.0f}" if tf else "", f"{tf / PEAK_TF:.3f}" if tf else ""])
    rows.append(["total", 86, f"{step:.1f}", "", "", "", ""])
    n = len(group)
    head = (f"{n} decode(s) of B={B} branches x T={T} rows, {S} steps: span {sum(spans) / n / 1e3:.2f} ms, "
            f"kernel-busy {sum(busy) / n / 1e3:.2f} ms per decode; one Euler step below (mean over them).\n\n")
    return head + md_table(["op", "launches/step", "us/step", "avg us/launch", "share", "TFLOP/s", "MFMA frac"],
                           rows), summary


def stats_table(path: Path, top: int = 16) -> str:
    rows = list(csv.DictReader(open(path)))
    body = [[r["Name"][:60], r["Calls"], f"{float(r['TotalDurationNs']) / 1e6:.2f}", f"{float(r['AverageNs']) / 1e3:.2f}",
             f"{float(r['MinNs']) / 1e3:.2f}", f"{float(r['MaxNs']) / 1e3:.2f}", f"{float(r['Percentage']):.2f}"]
            for r in rows[:top]]
    return md_table(["kernel", "calls", "total ms", "avg us", "min us", "max us", "%"], body)


def conv_roofline_loop(rows: list[dict], B: int = 2, T: int = 860) -> tuple | None:
    """The longest run of back-to-back k=5 conv GEMM launches at the decode shape
    (the bench's roofline timing loop), identified by the grid of the decode's
    conv launches."""
    grids = collections.Counter()
    for b_, t_, s_, seg in find_decodes(rows):
        if (b_, t_) == (B, T):
            for s in range(s_):
                for k, op in enumerate(STEP_ORDER):
                    if op == "conv":
                        r = seg[4 + s * 86 + k]
                        grids[(r["Grid_Size_X"], r["Workgroup_Size_X"])] += 1
    if not grids:
        return None
    g = grids.most_common(1)[0][0]
    best, i = (0, 0), 0
    while i < len(rows):
        if rows[i]["Kernel_Name"] == "gemm_kernel" and (rows[i]["Grid_Size_X"], rows[i]["Workgroup_Size_X"]) == g:
            j = i
            while j < len(rows) and rows[j]["Kernel_Name"] == "gemm_kernel" and \
                    (rows[j]["Grid_Size_X"], rows[j]["Workgroup_Size_X"]) == g:
                j += 1
            if j - i > best[1] - best[0]:
                best = (i, j)
            i = j
        else:
            i += 1
    d = [dur(r) for r in rows[best[0]:best[1]]]
    return (len(d), sum(d) / len(d), min(d), max(d), g) if d else None


# ---------------------------------------------------------------------------- condition producer
COND_NAMES = ["copy_prompt", "to_f16", "content_in_proj", "nearest_rows"]
COND_KERN = ["copyBuffer", "f32_to_f16_kernel", "gemm_kernel", "nearest_rows_kernel"]
for _b in range(4):
    COND_NAMES += [f"conv{_b}_k3", f"gn_mish{_b}"]
    COND_KERN += ["gemm_kernel", "gn_mish_kernel"]
COND_NAMES.append("out_conv_k1")
COND_KERN.append("gemm_kernel")


def condition_tables(rows: list[dict]) -> str:
    """Every condition-producer call (a prompt copy, then the length regulator's
    11 kernels), grouped by the grid signature of its GEMMs (the default split
    mode and the f16 mode launch different tilings)."""
    groups = collections.defaultdict(list)
    for i, r in enumerate(rows):
        n_call = len(COND_KERN)
        if "nearest_rows_kernel" not in r["Kernel_Name"] or i < 3 or i - 3 + n_call > len(rows):
            continue
        seg = rows[i - 3:i - 3 + n_call]
        if all(k in s["Kernel_Name"] for s, k in zip(seg, COND_KERN)):
            sig = tuple(s["Grid_Size_X"] for s in seg if "gemm_kernel" in s["Kernel_Name"])
            groups[sig].append(seg)
    out = []
    for sig, segs in sorted(groups.items(), key=lambda kv: -len(kv[1])):
        segs = segs[3:] if len(segs) > 6 else segs  # leave out the first calls (warm-up)
        n = len(segs)
        acc = [sum(dur(s[k]) for s in segs) / n for k in range(len(COND_NAMES))]
        tot = sum(acc)
        span = sum((int(s[-1]["End_Timestamp"]) - int(s[0]["Start_Timestamp"])) / 1000.0 for s in segs) / n
        body = [[n_, k_, f"{a:.2f}", f"{100 * a / tot:.1f}%"] for n_, k_, a in zip(COND_NAMES, COND_KERN, acc)]
        body.append(["total", "", f"{tot:.1f}", ""])
        out.append(f"### {n} calls, GEMM grids {', '.join(sig)}: mean span {span:.1f} us, kernel-busy {tot:.1f} us\n\n"
                   + md_table(["op", "kernel", "avg us", "share"], body))
    return "\n\n".join(out)


# ---------------------------------------------------------------------------- vocoder
def vocoder_tables(rows: list[dict], frames: int = 860) -> str:
    """Vocoder calls at `frames` mel frames: from the mel's f16 conversion
    (frames x 80 values) to the clamp of 256 x frames samples.  Grouped by the
    number of kernels per call (the same); the two modes come in order in the
    bench (default first, then f16), ten timed calls each after warm-ups."""
    calls, i = [], 0
    while i < len(rows):
        r = rows[i]
        if "f32_to_f16" in r["Kernel_Name"] and int(r["Grid_Size_X"]) == ((frames * 80 + 255) // 256) * 256:
            j = i
            while j < len(rows) and "conv_post_clamp" not in rows[j]["Kernel_Name"]:
                j += 1
            if j < len(rows) and int(rows[j]["Grid_Size_X"]) == frames * 256 and j - i < 400:
                calls.append((i, j))
                i = j
        i += 1

    def key(r):
        n = r["Kernel_Name"]
        for k in ("snake", "gemm_kernel", "conv_post_clamp", "f32_to_f16", "copy"):
            if k in n:
                return (k, r["Grid_Size_X"], r["Workgroup_Size_X"])
        return (n[:40], r["Grid_Size_X"], r["Workgroup_Size_X"])

    out = [f"vocoder calls at {frames} frames in the trace: {len(calls)}"]
    half = len(calls) // 2
    for name, cs in (("default (fp32-level) mode", calls[2:half]), ("f16 mode", calls[half + 2:])):
        if not cs:
            continue
        per, cnt = collections.defaultdict(float), collections.Counter()
        span = busy = 0.0
        for i, j in cs:
            span += (int(rows[j]["End_Timestamp"]) - int(rows[i]["Start_Timestamp"])) / 1000.0
            for r in rows[i:j + 1]:
                d = dur(r)
                per[key(r)] += d
                cnt[key(r)] += 1
                busy += d
        nc = len(cs)
        cls = collections.defaultdict(float)
        for k, v in per.items():
            cls[k[0]] += v / nc
        out.append(f"\n{name}: {nc} calls: span {span / nc:.1f} us, kernel-busy {busy / nc:.1f} us; by class "
                   + ", ".join(f"{k} {v:.1f} us" for k, v in cls.items()))
        for k in sorted(per, key=lambda k: -per[k]):
            out.append(f"  {per[k] / nc:8.1f} us/call  x{cnt[k] // nc:3d}  avg {per[k] / cnt[k]:7.2f}  {k}")
    return "\n".join(out)


# ---------------------------------------------------------------------------- counters
KERNELS = ["w13", "conv", "qkv", "w2", "attention", "adarms", "wo", "resskip"]  # profile_kernels.py order


def counter_table(raw: Path, fetch_factor: float, write_factor: float, N: int = 20) -> str | None:
    flops = {"w13": op_flops("w13", 2, 860), "conv": op_flops("conv", 2, 860), "qkv": op_flops("qkv", 2, 860),
             "w2": op_flops("w2", 2, 860), "attention": op_flops("attn", 2, 860), "adarms": 0.0,
             "wo": op_flops("wo", 2, 860), "resskip": op_flops("resskip", 2, 860)}
    res = collections.defaultdict(dict)
    for pas in PMC_PASSES:
        f = raw / f"pmc_{pas}" / "p_counter_collection.csv"
        if not f.exists():
            return None
        disp = collections.OrderedDict()
        for r in csv.DictReader(open(f)):
            d = int(r["Dispatch_Id"])
            disp.setdefault(d, {"t": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0,
                                "grid": int(r["Grid_Size"]), "wg": int(r["Workgroup_Size"])})
            disp[d][r["Counter_Name"]] = float(r["Counter_Value"])
        ids = sorted(disp)[-8 * N:]
        for k in range(8):
            sel = [disp[i] for i in ids[k * N + N // 2:(k + 1) * N]]  # the second half of each kernel's launches
            for c in sel[0]:
                v = sum(s[c] for s in sel) / len(sel)
                if c == "t":
                    res[KERNELS[k]].setdefault("t_list", []).append(v)
                else:
                    res[KERNELS[k]][c] = v
    body = []
    for k in KERNELS:
        r = res[k]
        t = sum(r["t_list"]) / len(r["t_list"])
        mf = flops[k] / (t * 1e-6) / (PEAK_TF * 1e12) if flops[k] else 0.0
        wait = r["SQ_WAIT_INST_ANY"] / r["SQ_WAVE_CYCLES"]
        hit = r["TCC_HIT_sum"] / max(r["TCC_HIT_sum"] + r["TCC_MISS_sum"], 1.0)
        lat = r["TCP_TCC_READ_REQ_LATENCY_sum"] / max(r["TCP_TCC_READ_REQ_sum"], 1.0)
        l2b = r["TCP_TCC_READ_REQ_sum"] * 128 / 1e6
        percu = r["TCP_TCC_READ_REQ_sum"] * 128 / 256 / t / 1e3
        hbm_r = r["FETCH_SIZE"] * fetch_factor / 1e6
        hbm_w = r["WRITE_SIZE"] * write_factor / 1e6
        body.append([k, f"{int(r['grid']) // int(r['wg'])} x {int(r['wg'])}", f"{t:.2f}", f"{mf:.3f}", f"{wait:.2f}",
                     f"{hit:.2f}", f"{lat:.0f}", f"{l2b:.1f}", f"{percu:.0f}", f"{hbm_r:.2f}", f"{hbm_w:.2f}",
                     f"{(hbm_r + hbm_w) / t:.2f}", f"{r['SQ_LDS_BANK_CONFLICT']:.0f}"])
    table = md_table(["kernel", "grid x wg", "us (pmc runs)", "MFMA frac", "wait share", "L2 hit",
                      "L2 read latency (cyc)", "L2->CU MB", "per-CU KB/us", "HBM read MB", "HBM write MB",
                      "HBM TB/s", "LDS bank conflicts"], body)
    keys = sorted(set().union(*[set(res[k]) for k in KERNELS]) - {"t_list", "grid", "wg"})
    raw_rows = [[c] + [f"{res[k].get(c, 0):.4g}" for k in KERNELS] for c in keys]
    return table, md_table(["counter"] + KERNELS, raw_rows)


def calibration(fetch_csv: Path, write_csv: Path, mib: int = 256) -> dict | None:
    """FETCH_SIZE / WRITE_SIZE of the bench's streaming copy (torch.mul over
    `mib` MiB: the largest elementwise dispatch of the run) and the bytes per
    KiB they imply."""
    if not (fetch_csv.exists() and write_csv.exists()):
        return None
    is_copy = lambda r: "elementwise" in r["Kernel_Name"]
    f = pmc_per_dispatch(fetch_csv, "FETCH_SIZE", is_copy)
    w = pmc_per_dispatch(write_csv, "WRITE_SIZE", is_copy)
    if not f or not w:
        return None
    fk, wk = max(f), max(w)
    b = mib * (1 << 20)
    return {"kernel": f"torch.mul(src, 1.0, out=dst) streaming copy, {mib} MiB read + {mib} MiB written",
            "fetch_size_kib": fk, "write_size_kib": wk,
            "fetch_factor_bytes_per_kib": round(b / fk, 2), "write_factor_bytes_per_kib": round(b / wk, 2)}


def pmc_per_dispatch(path: Path, counter: str, match) -> list[float]:
    vals = collections.defaultdict(float)
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] == counter and match(r):
            vals[int(r["Dispatch_Id"])] += float(r["Counter_Value"])
    return list(vals.values())


# ---------------------------------------------------------------------------- writers
def write_decode_profiles(raw: Path, out: Path) -> None:
    tr = raw / "trace" / "bench_kernel_trace.csv"
    if not tr.exists():
        print(f"skip decode tables: no {tr}")
        return
    rows = load_trace(tr)
    bt, bp = bench_line(raw / "trace.log"), bench_line(raw / "bench_plain.log")
    groups = collections.defaultdict(list)
    for B, T, S, seg in find_decodes(rows):
        groups[(B, T, S)].append(seg)
    stats = stats_table(raw / "trace" / "bench_kernel_stats.csv") if (raw / "trace" / "bench_kernel_stats.csv").exists() else ""
    loop = conv_roofline_loop(rows)
    head = f"""Commands (repo root, MI355X, one GPU):

```
{TRACE_CMD}
{PLAIN_CMD}
```
"""
    if bt and bp:
        head += (f"\nbench.py line of the traced run: value {bt['value']:,.1f} mel frames/s, {bt['ms_per_step']:.2f} ms per "
                 f"decode, decode MFMA util {bt['decode_mfma_util']:.3f}; roofline kernel avg "
                 f"{bt['roofline']['avg_launch_us']:.2f} us (HIP events), frac {bt['roofline']['frac']:.3f}.  "
                 f"Without the profiler, the run before on the same box: {bp['ms_per_step']:.2f} ms per decode, "
                 f"{bp['value']:,.1f} frames/s, roofline frac {bp['roofline']['frac']:.3f}.\n")
    if loop:
        head += (f"\nThe roofline kernel's timing loop in the trace ({loop[0]} back-to-back launches of the k=5 conv GEMM, "
                 f"grid {int(loop[4][0]):,} threads in workgroups of {loop[4][1]}): average {loop[1]:.2f} us, min "
                 f"{loop[2]:.2f}, max {loop[3]:.2f}.\n")
    key860 = (2, 860, 25)
    legend = """Ops are identified by their position in the captured step (86 dispatches after the decode's
four set-up dispatches).  TFLOP/s = algorithmic FLOPs per launch (model K: 80 mel columns for
`merge`, 592 for `post`) / average duration; MFMA frac against 2,500 TFLOP/s (f16 dense), at the
executed shape (B x T rows, padding included).  `fold` is block l's w2 folded with block l+1's
skip-in (blocks 6..11, K = 2560); `post` is conv1|res_projection with skip_linear folded in;
`finalskip` is the last WaveNet layer's res/skip GEMM (N = 512) with the res_projection add;
`conv2_euler` applies the final linear folded into conv2, the CFG blend and the Euler update."""
    if key860 in groups:
        t, _ = decode_table(groups[key860], *key860)
        md = (f"# DiT-CFM decode, T=860 (P=258), 25 steps, CFG 0.7, B=2 -- rocprofv3 kernel trace\n\n{head}\n"
              f"## rocprofv3 --stats (all dispatches of the run; -T truncates template names)\n\n{stats}\n\n"
              f"## Per op, one Euler step of the T=860 decode\n\n{legend}\n\n{t}\n")
        (out / "cfm_decode_T860_S25_B2_kernel_trace.md").write_text(md)
        print("wrote cfm_decode_T860_S25_B2_kernel_trace.md")
    known = [(2, 128, 12), (2, 3000, 25), (16, 1348, 16)]  # the other benchmark workloads with a decode
    others = [k for k in known if k in groups]
    if others:
        parts = []
        for B, T, S in others:
            segs = groups[(B, T, S)]
            what = {(2, 128, 12): "T=128 (P=48), 12 steps, B=2: the short-utterance workload",
                    (2, 3000, 25): "T=3000 (P=258), 25 steps, B=2: the long-form workload",
                    (16, 1348, 16): "8 right-padded requests (T_max=1348), 16 steps, B=16: the batched-serving workload"}
            title = what.get((B, T, S), f"B={B}, T={T}, {S} steps")
            if (B, T, S) == (16, 1348, 16) and bt:
                # the bench times this shape twice: padded rows computed, then skipped
                half = len(segs) // 2
                toks = bt.get("configs", {}).get("config5_8req_padded_B16_S16_skip_padding", {}).get("tokens")
                skip_fl = skipped_padding_flops(toks, T) if toks else None
                for label, ss, fl in (("padded rows computed", segs[:half], None),
                                      ("padded rows skipped (MIT2CFM_PADDING_SKIP)", segs[half:], skip_fl)):
                    if ss:
                        t, _ = decode_table(ss, B, T, S, fl)
                        parts.append(f"## {title}; {label}\n\n{t}")
            else:
                t, _ = decode_table(segs, B, T, S)
                parts.append(f"## {title}\n\n{t}")
        md = (f"# DiT-CFM decode at the other benchmark workloads -- rocprofv3 kernel trace\n\nThe same run as "
              f"profiles/cfm_decode_T860_S25_B2_kernel_trace.md.\n\n{head}\n{legend}  For the padded batch with its "
              f"padded rows computed the utilisation counts them, so it is the kernels' rate on the work they did; with "
              f"them skipped it counts the rows each product computes (each request's valid length + 2, both "
              f"branches) and, for the attention, those queries against the valid keys.  bench.py's "
              f"`decode_mfma_util` counts valid rows and keys only.\n\n" + "\n\n".join(parts) + "\n")
        (out / "cfm_decode_configs_kernel_trace.md").write_text(md)
        print("wrote cfm_decode_configs_kernel_trace.md")
    cond = condition_tables(rows)
    if cond and bp and "condition_producer" in bp:
        cp = bp["condition_producer"]
        md = f"""# Condition producer (length regulator 350 codes -> 602 frames + 258 prompt rows) -- rocprofv3 kernel trace

Same run as profiles/cfm_decode_T860_S25_B2_kernel_trace.md:

```
{TRACE_CMD}
```

bench.py `condition_producer` without the profiler: {cp['us_per_call']:.1f} us per call in the default mode (split f16
operand pairs, fp32-level products), f16 mode {cp.get('f16_mode', {}).get('us_per_call', float('nan')):.1f} us.  Each call is
`mit2cfm_condition_device`, replayed as one graph: a device copy of the 258 prompt rows, then the length regulator's
11 kernels (conv k=3 is the zero-padded implicit GEMM A_CONV3Z, M = 602, N = 512, K = 1536; gn_mish reduces the conv's
per-row partial sums in double, the same in every workgroup, then applies GroupNorm and Mish).  Groups below are the two precision modes (their GEMM grids differ).

{cond}
"""
        (out / "condition_producer_codes350_kernel_trace.md").write_text(md)
        print("wrote condition_producer_codes350_kernel_trace.md")
    voc = vocoder_tables(rows)
    if bp and "vocoder" in bp and "vocoder calls at 860 frames in the trace: 0" not in voc:
        vp = bp["vocoder"]
        md = f"""# BigVGAN vocoder, 860 mel frames -> 220,160 samples -- rocprofv3 kernel trace

Same run as profiles/cfm_decode_T860_S25_B2_kernel_trace.md:

```
{TRACE_CMD}
```

bench.py `vocoder` without the profiler: default (fp32-level) mode {vp['ms_per_call']:.3f} ms per call, f16 mode
{vp.get('f16_mode', {}).get('ms_per_call', float('nan')):.3f} ms.  `gemm_kernel` rows are the implicit-GEMM convs, keyed by
grid size and workgroup size: the 768- and 384-channel stages streaming every tap's rows (A_CONVP), the 192- to
24-channel stages and the upsamplers that read them with the row block's input window in LDS (A_CONVW); `snake` rows
are the anti-aliased SnakeBeta activations.  Algorithmic conv work: 1.551 TFLOP per call.

```
{voc}
```
"""
        (out / "bigvgan_T860_kernel_trace.md").write_text(md)
        print("wrote bigvgan_T860_kernel_trace.md")


def write_counter_profiles(raw: Path, out: Path) -> None:
    fe = raw / "pmc_bfetch" / "fetch_counter_collection.csv"
    wr = raw / "pmc_bwrite" / "write_counter_collection.csv"
    cal = calibration(fe, wr)
    ff = cal["fetch_factor_bytes_per_kib"] if cal else 2048.0
    wf = cal["write_factor_bytes_per_kib"] if cal else 1024.0
    tabs = counter_table(raw, ff, wf)
    if tabs:
        table, rawt = tabs
        cmds = "\n".join(f"rocprofv3 --pmc {c} --output-format csv -d $RAW/pmc_{p} -o p -- {PMC_PROG}"
                         for p, c in PMC_PASSES.items())
        md = f"""# Decode kernels at T=860 (M=1720) -- rocprofv3 counters

Five counter passes (one run each) over `index-tts2-metal_amd/profile_kernels.py`: one T=860
decode, then 20 back-to-back launches of each hot kernel at the decode's shape; each figure is
the mean over the last 10 launches of a kernel:

```
{cmds}
```

HBM bytes: FETCH_SIZE x {ff:.1f} and WRITE_SIZE x {wf:.1f} bytes per KiB, the factors the same counters give
for the bench's 256 MiB streaming copy (FETCH_SIZE counts half of what a copy reads on MI355X).  L2->CU
bytes: TCP_TCC_READ_REQ_sum x 128 B.  MFMA frac: algorithmic FLOPs / duration / 2,500 TFLOP/s.  Wait
share: SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES.

{table}

Raw counters (per dispatch):

{rawt}
"""
        (out / "decode_kernels_T860_counters.md").write_text(md)
        print("wrote decode_kernels_T860_counters.md")
    if cal:
        rows = load_trace(raw / "trace" / "bench_kernel_trace.csv") if (raw / "trace" / "bench_kernel_trace.csv").exists() else []
        loop = conv_roofline_loop(rows) if rows else None
        if loop:
            g = loop[4]
            match = lambda r: r["Kernel_Name"] == "gemm_kernel" and r["Grid_Size"] == g[0] and r["Workgroup_Size"] == g[1]
            f = pmc_per_dispatch(fe, "FETCH_SIZE", match)
            w = pmc_per_dispatch(wr, "WRITE_SIZE", match)
            if f and w:
                fk, wk = sum(f) / len(f), sum(w) / len(w)
                alg = 1720 * 512 * 2 + 1024 * 2560 * 2 + 1720 * 512 * 2 + 2048 * 4 + 1024 * 4
                j = {"kernel": "gemm_wavenet_conv_gate",
                     "workload": "WaveNet k=5 conv implicit GEMM + gate, M=1720 (B=2 x T=860), N=1024, K=2560",
                     "fetch_size_kib_per_dispatch": round(fk, 1), "write_size_kib_per_dispatch": round(wk, 1),
                     "calibration": cal, "hbm_bytes_per_launch": int(fk * ff + wk * wf),
                     "algorithmic_bytes_per_launch": alg,
                     "commands": [f"rocprofv3 --pmc FETCH_SIZE -T --output-format csv -d $RAW/pmc_bfetch -o fetch -- {BENCH_PMC}",
                                  f"rocprofv3 --pmc WRITE_SIZE -T --output-format csv -d $RAW/pmc_bwrite -o write -- {BENCH_PMC}"],
                     "dispatches_used": f"every dispatch of the conv GEMM at grid {g[0]} x {g[1]} in the runs ({len(f)}); "
                                        f"min/max FETCH_SIZE {min(f):.0f}/{max(f):.0f} KiB, WRITE_SIZE {min(w):.0f}/{max(w):.0f} KiB"}
                (out / "traffic_gemm_wavenet_conv_gate_T860.json").write_text(json.dumps(j, indent=1) + "\n")
                print("wrote traffic_gemm_wavenet_conv_gate_T860.json")


GPT_WHAT = {"c_attn": "c_attn GEMV 3840x1280 + LN, K/V to cache", "attn_proj": "attn c_proj GEMV 1280x1280 + residual",
            "c_fc": "c_fc GEMV 5120x1280 + LN + gelu_new", "mlp_proj": "mlp c_proj GEMV 1280x5120 + residual",
            "mel_head": "mel_head GEMV 8194x1280 + ln_f + final_norm"}
def gemv_roles(rows: list[dict], grid_key: str, wg_key: str) -> dict:
    """Kernel id -> product for the decode-step GEMVs, from their launch order
    within a layer (c_attn, the attention, attn c_proj, c_fc, mlp c_proj):
    two products can share a grid, so the grid alone does not name them.
    `rows` are dispatches in launch order."""
    g = [r for r in rows if "gemv_kernel" in r["Kernel_Name"] and "gemv_rows" not in r["Kernel_Name"]]
    roles = {}
    # attn c_proj is the GEMV launched right after an attention combine; the
    # first layer where the pattern is whole names all four
    seq = [r for r in rows if any(k in r["Kernel_Name"] for k in ("gemv_kernel", "attn_combine_kernel"))
           and "gemv_rows" not in r["Kernel_Name"]]
    for i in range(len(seq) - 3):
        if "attn_combine_kernel" in seq[i]["Kernel_Name"] and all("gemv_kernel" in seq[i + k]["Kernel_Name"]
                                                                   for k in (1, 2, 3)):
            roles.setdefault(seq[i + 1]["Kernel_Id"], "attn_proj")
            roles.setdefault(seq[i + 2]["Kernel_Id"], "c_fc")
            roles.setdefault(seq[i + 3]["Kernel_Id"], "mlp_proj")
            if i >= 1 and "gemv_kernel" in seq[i - 1]["Kernel_Name"]:
                roles.setdefault(seq[i - 1]["Kernel_Id"], "c_attn")
        if len(roles) >= 4:
            break
    for r in g:  # the head: the widest grid
        if int(r[grid_key]) // int(r[wg_key]) > 1000:
            roles.setdefault(r["Kernel_Id"], "mel_head")
    return roles


def gpt_kernel_key(r: dict, roles: dict) -> str:
    n = r["Kernel_Name"]
    for k in ("gemv_rows_kernel", "gemv_kernel", "attn_split_kernel", "attn_combine_kernel", "sample_kernel",
              "embed_rows_kernel", "embed_kernel", "argmax_kernel", "advance_rows_kernel"):
        if k in n:
            if k.startswith("gemv"):
                blocks = int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"])
                role = roles.get(r["Kernel_Id"]) if k == "gemv_kernel" else "prefill"
                return f"{k} {role or '?'} (grid {blocks}x{r['Workgroup_Size_X']})"
            return k
    return n[:40]


def write_gpt_profiles(raw: Path, out: Path) -> None:
    tr = raw / "gpttrace" / "bench_kernel_trace.csv"
    bt = bench_line(raw / "gpt_trace.log")
    if not tr.exists() or not bt or "gpt_decode" not in bt:
        print(f"skip GPT tables: no {tr} / gpt_trace.log")
        return
    rows = [r for r in load_trace(tr) if any(k in r["Kernel_Name"] for k in ("gemv", "attn_split", "attn_combine",
                                                                              "sample_kernel", "embed", "argmax",
                                                                              "advance_rows"))]
    roles = gemv_roles(rows, "Grid_Size_X", "Workgroup_Size_X")
    per = collections.defaultdict(list)
    for r in rows:
        per[gpt_kernel_key(r, roles)].append(dur(r))
    body = [[f"`{k}`", len(v), f"{sum(v) / len(v):.2f}", f"{min(v):.2f}", f"{max(v):.2f}", f"{sum(v) / 1e3:.2f}"]
            for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1]))]
    g = bt["gpt_decode"]
    # the c_fc timing loop: the longest run of back-to-back c_fc GEMVs
    best, i = (0, 0), 0
    key_fc = next((k for k in per if k.startswith("gemv_kernel c_fc ")), None)
    while i < len(rows):
        if gpt_kernel_key(rows[i], roles) == key_fc:
            j = i
            while j < len(rows) and gpt_kernel_key(rows[j], roles) == key_fc:
                j += 1
            if j - i > best[1] - best[0]:
                best = (i, j)
            i = j
        else:
            i += 1
    d = [dur(r) for r in rows[best[0]:best[1]]]
    loop = f"average {sum(d) / len(d):.2f} us, min {min(d):.2f}, max {max(d):.2f}" if d else "not found"
    cmds = "\n".join(GPT_CMDS)
    md = f"""# GPT mel-code decoder: 553 codes after a 150-row prefix, 24 layers -- rocprofv3 kernel trace

Commands (repo root, MI355X, one GPU).  The HIP-graph replay is switched off with MIT2CFM_GRAPH=0
(every kernel launched directly; the same kernels): one earlier kernel-trace run with graph replay
ended in a host SIGSEGV inside hipGraphLaunch of the GPT step graph.

```
{cmds}
```

bench.py `gpt_decode` of the traced run (direct launches, profiler attached): {g['ms_per_code']:.4f} ms per code, prefill
{g['prefill_ms']:.3f} ms.  Without the profiler and with graph replay the bench's figure is the one in the round's bench line.

## Per kernel (all dispatches of the GPT section; GEMVs named by product, with blocks x threads)

{md_table(['kernel', 'dispatches', 'avg us', 'min us', 'max us', 'total ms'], body)}

The roofline kernel's timing loop in this trace ({len(d)} back-to-back c_fc launches cycling the 24 layers'
weights): {loop} (kernel execution from the trace timestamps).
"""
    (out / "gpt_decode_P150_553codes_kernel_trace.md").write_text(md)
    print("wrote gpt_decode_P150_553codes_kernel_trace.md")
    fe = raw / "gptpmc_fetch" / "fetch_counter_collection.csv"
    wr = raw / "gptpmc_write" / "write_counter_collection.csv"
    cal = calibration(fe, wr)
    if cal:
        def fc_match(path: Path, counter: str):
            disp = {}
            for r in csv.DictReader(open(path)):
                if r["Counter_Name"] == counter:
                    disp.setdefault(int(r["Dispatch_Id"]), r)
            ordered = [disp[k] for k in sorted(disp)]
            fc = [k for k, v in gemv_roles(ordered, "Grid_Size", "Workgroup_Size").items() if v == "c_fc"]
            return lambda r: r["Kernel_Id"] in fc
        f = pmc_per_dispatch(fe, "FETCH_SIZE", fc_match(fe, "FETCH_SIZE"))
        w = pmc_per_dispatch(wr, "WRITE_SIZE", fc_match(wr, "WRITE_SIZE"))
        if f and w:
            fk, wk = sum(f) / len(f), sum(w) / len(w)
            j = {"kernel": "gemv_gpt_c_fc",
                 "workload": "GPT c_fc GEMV + LayerNorm prologue + gelu_new, 5120 x 1280 f16 weights, one 1280-wide input vector",
                 "fetch_size_kib_per_dispatch": round(fk, 1), "write_size_kib_per_dispatch": round(wk, 1),
                 "calibration": cal,
                 "hbm_bytes_per_launch": int(fk * cal["fetch_factor_bytes_per_kib"] + wk * cal["write_factor_bytes_per_kib"]),
                 "algorithmic_bytes_per_launch": 5120 * 1280 * 2 + 1280 * 4 * 3 + 5120 * 4 * 2,
                 "commands": GPT_CMDS[1:],
                 "dispatches_used": f"every dispatch of the c_fc GEMV in the runs ({len(f)}); min/max FETCH_SIZE "
                                    f"{min(f):.0f}/{max(f):.0f} KiB"}
            (out / "traffic_gemv_gpt_c_fc.json").write_text(json.dumps(j, indent=1) + "\n")
            print("wrote traffic_gemv_gpt_c_fc.json")


def unpack_raw(raw: Path) -> None:
    """Raw CSVs may arrive gzip-compressed (NAME.csv.gz, to keep a run's output
    small); each is unpacked beside itself once."""
    for gz in sorted(raw.rglob("*.csv.gz")):
        dst = gz.with_suffix("")
        if not dst.exists():
            with gzip.open(gz, "rb") as f, open(dst, "wb") as o:
                shutil.copyfileobj(f, o)


def main() -> None:
    root = Path(__file__).resolve().parent.parent
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--raw", type=Path, required=True, help="directory of the rocprofv3 output")
    p.add_argument("--out", type=Path, default=root / "profiles", help="where the summaries go")
    a = p.parse_args()
    a.out.mkdir(parents=True, exist_ok=True)
    unpack_raw(a.raw)
    write_decode_profiles(a.raw, a.out)
    write_counter_profiles(a.raw, a.out)
    write_gpt_profiles(a.raw, a.out)


if __name__ == "__main__":
    main()
