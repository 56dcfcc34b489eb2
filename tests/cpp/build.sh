#!/bin/sh
# Builds tests/cpp/dropin_link against the in-tree headers and unholy_amd/libunholy_amd.so (gfx950). Usage:
#   tests/cpp/build.sh [output]      (default: tests/cpp/dropin_link)
set -e
here=$(cd "$(dirname "$0")" && pwd)
root=$(cd "$here/../.." && pwd)
out=${1:-$here/dropin_link}
"${HIPCC:-/opt/rocm/bin/hipcc}" --offload-arch=gfx950 -O2 -std=c++20 -I "$root/include" "$here/dropin_link.cpp" \
  -L "$root/unholy_amd" -lunholy_amd -Wl,-rpath,'$ORIGIN/../../unholy_amd' -o "$out"
