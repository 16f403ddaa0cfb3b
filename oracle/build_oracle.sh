#!/usr/bin/env bash
# Builds the scalar C restatement (test infrastructure) into oracle/liboracle.so.
# Plain IEEE arithmetic: no -ffast-math, no FMA contraction.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
gcc -O2 -fPIC -shared -std=c11 -ffp-contract=off -fno-fast-math \
    -o "$here/liboracle.so.tmp" "$here/tkv_oracle.c" -lm
mv -f "$here/liboracle.so.tmp" "$here/liboracle.so"
