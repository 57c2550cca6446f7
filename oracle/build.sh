#!/bin/sh
# Builds the CPU oracle (test infrastructure only) into oracle/liboracle.so.
# -ffp-contract=off -fno-fast-math keep fp32 operations separate and ordered,
# like the reference's scalar Swift CPU path (src/Check.swift:393-494).
# The reference itself (Swift + Metal) cannot be compiled in this image, so
# there is no oracle/_ref build.
set -e
here=$(cd "$(dirname "$0")" && pwd)
gcc -O2 -ffp-contract=off -fno-fast-math -fPIC -shared -std=c11 -Wall -Wextra \
    "$here/oracle.c" -o "$here/liboracle.so.tmp" -lm
mv "$here/liboracle.so.tmp" "$here/liboracle.so"
