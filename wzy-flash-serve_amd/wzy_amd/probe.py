"""Drive the BASELINE config-4 stage in one mode for profiling (rocprofv3 --kernel-trace / --pmc):

  python -m wzy_amd.probe step   N   N single-token decode steps at a 32K-cell prefilled context
  python -m wzy_amd.probe window N   N T=4 verify windows (snapshots on, commit of row 0 after each)
  python -m wzy_amd.probe mtp    N   N drafter steps (114,452-row draft head) after one decode step

Kernels are launched directly (no graph replay) unless --graphs is given.  Each unit prints its
wall time, so a trace can be read per unit.
"""
import argparse
import os
import sys
import time

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import numpy as np  # noqa: E402

import wzy_amd  # noqa: E402


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("mode", choices=("step", "window", "mtp"))
    ap.add_argument("n", type=int)
    ap.add_argument("--n-ctx", type=int, default=32768)
    ap.add_argument("--graphs", action="store_true")
    ap.add_argument("--warmup", type=int, default=2)
    args = ap.parse_args()
    wz = wzy_amd.lib()
    wz.wzy_dev_set(0)
    cfg = wzy_amd.default_cfg(args.n_ctx + 8 * (args.n + args.warmup) + 64)
    st = wzy_amd.Stage(cfg)
    wz.wzy_stage_set_graphs(st.h, 1 if args.graphs else 0)
    st.load_synthetic(3, args.n_ctx)
    rng = np.random.default_rng(1)
    pos = args.n_ctx
    if args.mode == "mtp":
        st.mtp_init(4, 114452)
        st.forward(pos, [5])
        st.sync()
    for i in range(args.warmup + args.n):
        t0 = time.perf_counter()
        if args.mode == "step":
            st.forward(pos, [int(rng.integers(0, cfg.n_vocab))])
            st.sync()
            pos += 1
        elif args.mode == "window":
            st.forward(pos, [int(x) for x in rng.integers(0, cfg.n_vocab, 4)], save_snaps=True)
            st.sync()
            st.lib.wzy_stage_commit_window_state(st.h, 0, pos)
            st.sync()
            pos += 1
        else:
            st.mtp_draft(pos, 7, 0, 1)
        print("%s %d %.3f ms%s" % (args.mode, i, 1000 * (time.perf_counter() - t0),
                                   " (warm-up)" if i < args.warmup else ""), flush=True)
    st.close()
    print("done", flush=True)


if __name__ == "__main__":
    main()
