#!/usr/bin/env bash
# rocprofv3 profile of every entry point at one N (the reference's bench/profile.sh used Nsight
# Compute / Nsight Systems): a kernel trace with per-kernel statistics, then one counter pass per
# group (rocprofv3 does not split counters over passes; each group fits the per-block limits).
#
#   bash phantom-a100_amd/bench/profile.sh            # N = 4096, output under gpurun_out/profile
#   N=8192 OUT=/tmp/prof bash phantom-a100_amd/bench/profile.sh
set -euo pipefail
HERE="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
N="${N:-4096}"
OUT="${OUT:-$PWD/gpurun_out/profile}"
mkdir -p "$OUT"
export TMPDIR=/tmp
PASS_A="SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT GRBM_GUI_ACTIVE"
PASS_B="SQ_ACTIVE_INST_VALU SQ_WAIT_INST_ANY SQ_LDS_IDX_ACTIVE SQ_INSTS_SALU GRBM_GUI_ACTIVE"
for impl in naive tiled fused fused_vec fused_db fused_tc; do
  echo "== $impl (N=$N)"
  timeout -k 10 300 rocprofv3 --kernel-trace --stats --output-format csv -d "$OUT/$impl/trace" -o trace -- \
    python3 "$HERE/run_one.py" --impl "$impl" --n "$N"
  i=0
  for pass in FETCH_SIZE WRITE_SIZE "$PASS_A" "$PASS_B"; do
    i=$((i + 1))
    # shellcheck disable=SC2086
    timeout -s KILL 120 rocprofv3 --pmc $pass --output-format csv -d "$OUT/$impl/pmc$i" -o pmc$i -- \
      python3 "$HERE/run_one.py" --impl "$impl" --n "$N" --reps 3
  done
done
echo "done: $OUT"
