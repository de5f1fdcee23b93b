// Drop-in include name: a reference caller (nirw4nna/hipgemm test.cpp:1,
// bench.cpp:1) that does `#include "fp8_4wave.hpp"` compiles unchanged against
// this library with `-I<repo>/include`.
#pragma once
#include "hipgemm/fp8_gemm.hpp"
