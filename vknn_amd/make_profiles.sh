#!/bin/bash
# Regenerates the rocprofv3 summaries under profiles/ on a GPU box, all on the plan file that
# bench.py reads by default (profiles/bench_plans.vkc), so every figure of the bench line can be
# recomputed from a summary of the same plans. Writes the new summaries to $OUT (default
# gpurun_out/profiles); copy them into profiles/ afterwards.
#   make_profiles.sh [--retune]   --retune: delete the plan file first and let one full bench run
#                                 re-tune every session of the bench (and write the file anew)
set -e -o pipefail
R=$(cd "$(dirname "$0")/.." && pwd)
OUT=${OUT:-$R/gpurun_out/profiles}
T=${TMPDIR:-/tmp}/vknn_prof
mkdir -p "$OUT" "$T"
cd /tmp && export TMPDIR=/tmp
PLANS=$R/profiles/bench_plans.vkc
if [ "$1" = "--retune" ]; then
    rm -f "$PLANS"
    echo "[make_profiles] tuning every bench session into $PLANS" >&2
    timeout -k 10 900 python3 "$R/bench.py" --plans "$PLANS" --steps 5 --warmup 2 --no-cpu-baseline > "$OUT/retune_bench.json" 2> "$OUT/retune_bench.log"
    cp "$PLANS" "$OUT/bench_plans.vkc"
fi
# the counter calibration: a flat fp32 -> fp16 convert of known traffic
timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE --output-format csv -d "$T/cal_f" -o run -- python3 "$R/bench.py" --traffic-probe 64 > /dev/null 2>&1
timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE --output-format csv -d "$T/cal_w" -o run -- python3 "$R/bench.py" --traffic-probe 64 > /dev/null 2>&1
python3 - "$T" > "$OUT/calibration.txt" <<'PY'
import csv, sys
t = sys.argv[1]
for c, d in (("FETCH_SIZE", "cal_f"), ("WRITE_SIZE", "cal_w")):
    v = [float(r["Counter_Value"]) for r in csv.DictReader(open(f"{t}/{d}/run_counter_collection.csv"))
         if r["Counter_Name"] == c and "pack_flat" in r["Kernel_Name"]]
    print(c, "KiB per launch of pack_flat_kernel (256 MB read, 128 MB written):", round(sum(v) / len(v)))
PY
# workload: stem model batch options title
prof() {
    local stem=$1 model=$2 batch=$3 extra=$4 title=$5
    local C="--plans $PLANS --model $model --batch $batch --steps 10 --warmup 2 --b1-steps 0 --no-profile --no-cpu-baseline --no-configs --dw-batch 0"
    local O="branches=0${extra:+;$extra}"
    echo "[make_profiles] $stem" >&2
    VKNN_HIP_OP_MARKERS=1 timeout -s KILL 300 rocprofv3 --kernel-trace --stats --output-format csv -d "$T/$stem" -o run -- \
        python3 "$R/bench.py" $C --options "$O" --plan-out "$T/$stem.plan" > "$T/$stem.log" 2>&1
    VKNN_HIP_OP_MARKERS=1 timeout -s KILL 300 rocprofv3 --pmc FETCH_SIZE --output-format csv -d "$T/${stem}_f" -o run -- \
        python3 "$R/bench.py" $C --options "$O" > /dev/null 2>&1
    VKNN_HIP_OP_MARKERS=1 timeout -s KILL 300 rocprofv3 --pmc WRITE_SIZE --output-format csv -d "$T/${stem}_w" -o run -- \
        python3 "$R/bench.py" $C --options "$O" > /dev/null 2>&1
    local cmd="VKNN_HIP_OP_MARKERS=1 rocprofv3 --kernel-trace --stats (then --pmc FETCH_SIZE, then --pmc WRITE_SIZE) -- python3 bench.py ${C//$R\//} --options \"$O\" --plan-out plan.txt; python3 -m vknn_amd.prof_summary layers|trace ... --steps 10 --fetch-scale 2 --write-scale 1"
    PYTHONPATH="$R" python3 -m vknn_amd.prof_summary layers "$T/$stem/run_kernel_trace.csv" "$T/$stem.plan" --steps 10 \
        --fetch "$T/${stem}_f/run_counter_collection.csv" --write "$T/${stem}_w/run_counter_collection.csv" --fetch-scale 2 --write-scale 1 \
        --title "$title: per-layer roofline on MI355X" --command "$cmd" > "$OUT/${stem}_layers.md"
    PYTHONPATH="$R" python3 -m vknn_amd.prof_summary trace "$T/$stem/run_kernel_trace.csv" --steps 10 \
        --title "$title: kernel time per step on MI355X" --command "$cmd" > "$OUT/${stem}_kernels.md"
    PYTHONPATH="$R" python3 -m vknn_amd.prof_summary traffic "$T/${stem}_f/run_counter_collection.csv" "$T/${stem}_w/run_counter_collection.csv" \
        --steps 10 --fetch-scale 2 --write-scale 1 --title "$title: HBM traffic per kernel family on MI355X" --command "$cmd" > "$OUT/${stem}_traffic.md"
    grep "b$batch:" "$T/$stem.log" >> "$OUT/${stem}_kernels.md" || true
    if [ -n "$STALLS" ]; then
        # wave states: two counter passes on the same plans (SQ_WAVE_CYCLES in both as the denominator)
        timeout -s KILL 300 rocprofv3 --pmc SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_VMEM SQ_ACTIVE_INST_LDS SQ_ACTIVE_INST_SCA \
            --output-format csv -d "$T/${stem}_sa" -o run -- python3 "$R/bench.py" $C --options "$O" > /dev/null 2>&1
        timeout -s KILL 300 rocprofv3 --pmc SQ_WAVE_CYCLES SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_LDS_BANK_CONFLICT SQ_VMEM_TA_ADDR_FIFO_FULL SQ_INSTS_VALU SQ_WAVES \
            --output-format csv -d "$T/${stem}_sb" -o run -- python3 "$R/bench.py" $C --options "$O" > /dev/null 2>&1
        PYTHONPATH="$R" python3 -m vknn_amd.prof_summary stalls "$T/${stem}_sa/run_counter_collection.csv" "$T/${stem}_sb/run_counter_collection.csv" --steps 10 \
            --title "$title: wave states and MFMA busy per kernel family on MI355X" \
            --command "rocprofv3 --pmc SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_VMEM SQ_ACTIVE_INST_LDS SQ_ACTIVE_INST_SCA, then --pmc SQ_WAVE_CYCLES SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_LDS_BANK_CONFLICT SQ_VMEM_TA_ADDR_FIFO_FULL SQ_INSTS_VALU SQ_WAVES -- python3 bench.py ${C//$R\//} --options \"$O\"; python3 -m vknn_amd.prof_summary stalls ... --steps 10" \
            > "$OUT/${stem}_stalls.md"
    fi
}
for w in ${WORKLOADS:-resnet50_b64 resnet50_b1 mobilenetv3_large_b128 yolov8n_b16 mnv2_block_b128 mnv2_block_b32 conv3x3_bn_relu_b1}; do
    case $w in
        resnet50_b64) STALLS=1 prof $w resnet50 64 "" "ResNet-50 b64 forward (config 2)" ;;
        resnet50_b1) prof $w resnet50 1 "" "ResNet-50 b1 forward (config 2)" ;;
        mobilenetv3_large_b128) STALLS=1 prof $w mobilenetv3_large 128 "" "MobileNetV3-Large b128 forward (config 3)" ;;
        yolov8n_b16) prof $w yolov8n 16 "" "YOLOv8n b16 forward (config 4)" ;;
        mnv2_block_b128) prof $w mnv2_block 128 "fuse_dwpw=1" "MobileNetV2 block b128 with the dw+pw fusion (config 1)" ;;
        mnv2_block_b32) prof $w mnv2_block 32 "" "MobileNetV2 block b32 (config 1)" ;;
        conv3x3_bn_relu_b1) prof $w conv3x3_bn_relu 1 "" "Conv3x3 + BN + ReLU b1 (config 0)" ;;
    esac
done
cp "$PLANS" "$OUT/bench_plans.vkc" 2>/dev/null || true
echo "[make_profiles] done" >&2
