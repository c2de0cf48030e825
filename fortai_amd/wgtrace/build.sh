#!/bin/bash
# Build the per-workgroup timing variant of libfortai_hip.so into
# fortai_amd/wgtrace/libfortai_wgtrace.so: the decode kernels' sources with
# trace.h force-included (the other objects are the library's own, so build
# the library first: python -c "from fortai_amd import build; build.build()").
# run.py reads the single-sequence decode step with it, run_batch.py the
# batch-8 step.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
F="--offload-arch=gfx950 -O3 -std=c++17 -fPIC -ffp-contract=off -Xclang -target-feature -Xclang -packed-fp32-ops"
OBJ="$HERE/obj"
mkdir -p "$OBJ"
objs=""
for f in "$ROOT"/fortai_amd/csrc/*.hip; do
  b=$(basename "$f" .hip)
  case $b in
    q8_kernels|gdn|attention|lm_head)
      printf '#include "%s"\nFORTAI_WGTRACE_EXPORT(%s)\n' "$f" "$b" > "$OBJ/$b.tu.hip"
      /opt/rocm/bin/hipcc $F -include "$HERE/trace.h" -I "$ROOT/fortai_amd/csrc" -c "$OBJ/$b.tu.hip" -o "$OBJ/$b.o" &
      objs="$objs $OBJ/$b.o";;
    *) objs="$objs $ROOT/fortai_amd/lib/obj/$b.o";;
  esac
done
wait
/opt/rocm/bin/hipcc --offload-arch=gfx950 -shared -fPIC $objs -o "$HERE/libfortai_wgtrace.so"
