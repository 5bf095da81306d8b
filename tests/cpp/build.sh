#!/bin/sh
# Builds tests/cpp/engine_abi (a C++ caller of the library's C ABI, checked against the CPU oracle) from the
# repository root; run after the library and the oracle are built (__graft_entry__.build() does all three).
set -e
cd "$(dirname "$0")/../.."
hipcc -O2 -std=c++17 -Iinclude -Ioracle tests/cpp/engine_abi.cpp -o tests/cpp/engine_abi \
  -Lr4dx_amd -lr4d_mi355x -Loracle/_build -lr4o \
  -Wl,-rpath,'$ORIGIN/../../r4dx_amd' -Wl,-rpath,'$ORIGIN/../../oracle/_build'
