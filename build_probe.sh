#!/bin/bash
# builds probe libraries with timing switches
set -e
cd "$(dirname "$0")/probe_csrc"
H=/opt/rocm/bin/hipcc
F="--offload-arch=gfx950 -O3 -std=c++17 -fPIC -ffp-contract=off -Xclang -target-feature -Xclang -packed-fp32-ops"
$H $F -c gossmx_api.hip -o api.o 2>/dev/null
for v in base:"" nocompute:"-DPROBE_NOCOMPUTE=1" nodma:"-DPROBE_NODMA=1" nobarrier:"-DPROBE_NOBARRIER=1" nodma_nobar:"-DPROBE_NODMA=1 -DPROBE_NOBARRIER=1" nocomp_nodma:"-DPROBE_NOCOMPUTE=1 -DPROBE_NODMA=1"; do
  name=${v%%:*}; defs=${v#*:}
  $H $F $defs -c gossmx_kernels.hip -o k_$name.o 2>/dev/null
  $H --offload-arch=gfx950 -shared -fPIC -o ../lib_$name.so k_$name.o api.o
done
