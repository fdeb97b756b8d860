#!/bin/sh
# Compile one of the reference's single-file CPU torch extensions (race_pref.cpp,
# linear_pref.cpp) where it lies, as an extra checker in oracle/_ref (never shipped
# as product, never copied).
# usage: build_ref.sh <path/to/source.cpp> <out.so> <extension name>
set -e
SRC="$1"; OUT="$2"; NAME="${3:-race_pref_ref}"
mkdir -p "$(dirname "$OUT")"
TI=$(python3 -c "import torch,os;print(os.path.dirname(torch.__file__))")
PYI=$(python3 -c "import sysconfig;print(sysconfig.get_paths()['include'])")
ABI=$(python3 -c "import torch;print(int(torch._C._GLIBCXX_USE_CXX11_ABI))")
g++ -O3 -fopenmp -shared -fPIC -std=c++17 \
  -DTORCH_EXTENSION_NAME=$NAME -DTORCH_API_INCLUDE_EXTENSION_H \
  -D_GLIBCXX_USE_CXX11_ABI=$ABI \
  -I"$TI/include" -I"$TI/include/torch/csrc/api/include" -I"$PYI" \
  "$SRC" -L"$TI/lib" -lc10 -ltorch -ltorch_cpu -ltorch_python \
  -Wl,-rpath,"$TI/lib" -o "$OUT"
echo "built $OUT"
