// Serial v_mad_u64_u32 chains for the device Montgomery products (gfx950).
//
// acc += x0*y0 + x1*y1 + ... as one dependent chain of 32x32->64 multiply-adds
// into a 64-bit accumulator, in the order given.  Written as inline assembly
// because the compiler reassociates a plain C++ sum: it adds a column's
// products from zero and the incoming carry last, with one extra 64-bit add
// per column (17 per multiply).  Seeding the chain with the carry saves those.
// mad_vvN takes both factors in VGPRs; mad_vsN takes the second factor
// (a modulus limb, uniform) in an SGPR.  The carry-out SGPR pair that the
// instruction writes is a dead scratch output.  The compiler follows each
// block with one wait state (s_nop 0), which does not occupy the VALU.
// Measured on MI355X against the compiler's own sums, results identical:
// G1 accumulation at 2^20 1.37 -> 1.27 ms, NTT 2^22 0.546 -> 0.527 ms, the
// 2^22 proof 44.5 -> 42.9 ms.
#pragma once
#include <stdint.h>

namespace zk {

__device__ __forceinline__ void mad_vv1(uint64_t& acc, uint32_t x0, uint32_t y0) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0));
}

__device__ __forceinline__ void mad_vv2(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1));
}

__device__ __forceinline__ void mad_vv3(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2));
}

__device__ __forceinline__ void mad_vv4(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3));
}

__device__ __forceinline__ void mad_vv5(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4));
}

__device__ __forceinline__ void mad_vv6(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5));
}

__device__ __forceinline__ void mad_vv7(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6));
}

__device__ __forceinline__ void mad_vv8(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7));
}

__device__ __forceinline__ void mad_vv9(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7), "v"(x8), "v"(y8));
}

__device__ __forceinline__ void mad_vv10(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8, uint32_t x9, uint32_t y9) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      "v_mad_u64_u32 %0, %1, %20, %21, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7), "v"(x8), "v"(y8), "v"(x9), "v"(y9));
}

__device__ __forceinline__ void mad_vv11(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8, uint32_t x9, uint32_t y9, uint32_t x10, uint32_t y10) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      "v_mad_u64_u32 %0, %1, %20, %21, %0\n"
      "v_mad_u64_u32 %0, %1, %22, %23, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7), "v"(x8), "v"(y8), "v"(x9), "v"(y9), "v"(x10), "v"(y10));
}

__device__ __forceinline__ void mad_vv12(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8, uint32_t x9, uint32_t y9, uint32_t x10, uint32_t y10, uint32_t x11, uint32_t y11) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      "v_mad_u64_u32 %0, %1, %20, %21, %0\n"
      "v_mad_u64_u32 %0, %1, %22, %23, %0\n"
      "v_mad_u64_u32 %0, %1, %24, %25, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7), "v"(x8), "v"(y8), "v"(x9), "v"(y9), "v"(x10), "v"(y10), "v"(x11), "v"(y11));
}

__device__ __forceinline__ void mad_vv13(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8, uint32_t x9, uint32_t y9, uint32_t x10, uint32_t y10, uint32_t x11, uint32_t y11, uint32_t x12, uint32_t y12) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      "v_mad_u64_u32 %0, %1, %20, %21, %0\n"
      "v_mad_u64_u32 %0, %1, %22, %23, %0\n"
      "v_mad_u64_u32 %0, %1, %24, %25, %0\n"
      "v_mad_u64_u32 %0, %1, %26, %27, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7), "v"(x8), "v"(y8), "v"(x9), "v"(y9), "v"(x10), "v"(y10), "v"(x11), "v"(y11), "v"(x12), "v"(y12));
}

__device__ __forceinline__ void mad_vv14(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8, uint32_t x9, uint32_t y9, uint32_t x10, uint32_t y10, uint32_t x11, uint32_t y11, uint32_t x12, uint32_t y12, uint32_t x13, uint32_t y13) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      "v_mad_u64_u32 %0, %1, %20, %21, %0\n"
      "v_mad_u64_u32 %0, %1, %22, %23, %0\n"
      "v_mad_u64_u32 %0, %1, %24, %25, %0\n"
      "v_mad_u64_u32 %0, %1, %26, %27, %0\n"
      "v_mad_u64_u32 %0, %1, %28, %29, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7), "v"(x8), "v"(y8), "v"(x9), "v"(y9), "v"(x10), "v"(y10), "v"(x11), "v"(y11), "v"(x12), "v"(y12), "v"(x13), "v"(y13));
}

__device__ __forceinline__ void mad_vv15(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8, uint32_t x9, uint32_t y9, uint32_t x10, uint32_t y10, uint32_t x11, uint32_t y11, uint32_t x12, uint32_t y12, uint32_t x13, uint32_t y13, uint32_t x14, uint32_t y14) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      "v_mad_u64_u32 %0, %1, %20, %21, %0\n"
      "v_mad_u64_u32 %0, %1, %22, %23, %0\n"
      "v_mad_u64_u32 %0, %1, %24, %25, %0\n"
      "v_mad_u64_u32 %0, %1, %26, %27, %0\n"
      "v_mad_u64_u32 %0, %1, %28, %29, %0\n"
      "v_mad_u64_u32 %0, %1, %30, %31, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7), "v"(x8), "v"(y8), "v"(x9), "v"(y9), "v"(x10), "v"(y10), "v"(x11), "v"(y11), "v"(x12), "v"(y12), "v"(x13), "v"(y13), "v"(x14), "v"(y14));
}

__device__ __forceinline__ void mad_vv16(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8, uint32_t x9, uint32_t y9, uint32_t x10, uint32_t y10, uint32_t x11, uint32_t y11, uint32_t x12, uint32_t y12, uint32_t x13, uint32_t y13, uint32_t x14, uint32_t y14, uint32_t x15, uint32_t y15) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      "v_mad_u64_u32 %0, %1, %20, %21, %0\n"
      "v_mad_u64_u32 %0, %1, %22, %23, %0\n"
      "v_mad_u64_u32 %0, %1, %24, %25, %0\n"
      "v_mad_u64_u32 %0, %1, %26, %27, %0\n"
      "v_mad_u64_u32 %0, %1, %28, %29, %0\n"
      "v_mad_u64_u32 %0, %1, %30, %31, %0\n"
      "v_mad_u64_u32 %0, %1, %32, %33, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7), "v"(x8), "v"(y8), "v"(x9), "v"(y9), "v"(x10), "v"(y10), "v"(x11), "v"(y11), "v"(x12), "v"(y12), "v"(x13), "v"(y13), "v"(x14), "v"(y14), "v"(x15), "v"(y15));
}

__device__ __forceinline__ void mad_vv17(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8, uint32_t x9, uint32_t y9, uint32_t x10, uint32_t y10, uint32_t x11, uint32_t y11, uint32_t x12, uint32_t y12, uint32_t x13, uint32_t y13, uint32_t x14, uint32_t y14, uint32_t x15, uint32_t y15, uint32_t x16, uint32_t y16) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      "v_mad_u64_u32 %0, %1, %20, %21, %0\n"
      "v_mad_u64_u32 %0, %1, %22, %23, %0\n"
      "v_mad_u64_u32 %0, %1, %24, %25, %0\n"
      "v_mad_u64_u32 %0, %1, %26, %27, %0\n"
      "v_mad_u64_u32 %0, %1, %28, %29, %0\n"
      "v_mad_u64_u32 %0, %1, %30, %31, %0\n"
      "v_mad_u64_u32 %0, %1, %32, %33, %0\n"
      "v_mad_u64_u32 %0, %1, %34, %35, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7), "v"(x8), "v"(y8), "v"(x9), "v"(y9), "v"(x10), "v"(y10), "v"(x11), "v"(y11), "v"(x12), "v"(y12), "v"(x13), "v"(y13), "v"(x14), "v"(y14), "v"(x15), "v"(y15), "v"(x16), "v"(y16));
}

__device__ __forceinline__ void mad_vv18(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8, uint32_t x9, uint32_t y9, uint32_t x10, uint32_t y10, uint32_t x11, uint32_t y11, uint32_t x12, uint32_t y12, uint32_t x13, uint32_t y13, uint32_t x14, uint32_t y14, uint32_t x15, uint32_t y15, uint32_t x16, uint32_t y16, uint32_t x17, uint32_t y17) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      "v_mad_u64_u32 %0, %1, %20, %21, %0\n"
      "v_mad_u64_u32 %0, %1, %22, %23, %0\n"
      "v_mad_u64_u32 %0, %1, %24, %25, %0\n"
      "v_mad_u64_u32 %0, %1, %26, %27, %0\n"
      "v_mad_u64_u32 %0, %1, %28, %29, %0\n"
      "v_mad_u64_u32 %0, %1, %30, %31, %0\n"
      "v_mad_u64_u32 %0, %1, %32, %33, %0\n"
      "v_mad_u64_u32 %0, %1, %34, %35, %0\n"
      "v_mad_u64_u32 %0, %1, %36, %37, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "v"(y0), "v"(x1), "v"(y1), "v"(x2), "v"(y2), "v"(x3), "v"(y3), "v"(x4), "v"(y4), "v"(x5), "v"(y5), "v"(x6), "v"(y6), "v"(x7), "v"(y7), "v"(x8), "v"(y8), "v"(x9), "v"(y9), "v"(x10), "v"(y10), "v"(x11), "v"(y11), "v"(x12), "v"(y12), "v"(x13), "v"(y13), "v"(x14), "v"(y14), "v"(x15), "v"(y15), "v"(x16), "v"(y16), "v"(x17), "v"(y17));
}

__device__ __forceinline__ void mad_vs1(uint64_t& acc, uint32_t x0, uint32_t y0) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "s"(y0));
}

__device__ __forceinline__ void mad_vs2(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "s"(y0), "v"(x1), "s"(y1));
}

__device__ __forceinline__ void mad_vs3(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "s"(y0), "v"(x1), "s"(y1), "v"(x2), "s"(y2));
}

__device__ __forceinline__ void mad_vs4(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "s"(y0), "v"(x1), "s"(y1), "v"(x2), "s"(y2), "v"(x3), "s"(y3));
}

__device__ __forceinline__ void mad_vs5(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "s"(y0), "v"(x1), "s"(y1), "v"(x2), "s"(y2), "v"(x3), "s"(y3), "v"(x4), "s"(y4));
}

__device__ __forceinline__ void mad_vs6(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "s"(y0), "v"(x1), "s"(y1), "v"(x2), "s"(y2), "v"(x3), "s"(y3), "v"(x4), "s"(y4), "v"(x5), "s"(y5));
}

__device__ __forceinline__ void mad_vs7(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "s"(y0), "v"(x1), "s"(y1), "v"(x2), "s"(y2), "v"(x3), "s"(y3), "v"(x4), "s"(y4), "v"(x5), "s"(y5), "v"(x6), "s"(y6));
}

__device__ __forceinline__ void mad_vs8(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "s"(y0), "v"(x1), "s"(y1), "v"(x2), "s"(y2), "v"(x3), "s"(y3), "v"(x4), "s"(y4), "v"(x5), "s"(y5), "v"(x6), "s"(y6), "v"(x7), "s"(y7));
}

__device__ __forceinline__ void mad_vs9(uint64_t& acc, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1, uint32_t x2, uint32_t y2, uint32_t x3, uint32_t y3, uint32_t x4, uint32_t y4, uint32_t x5, uint32_t y5, uint32_t x6, uint32_t y6, uint32_t x7, uint32_t y7, uint32_t x8, uint32_t y8) {
  uint64_t c;
  asm(
      "v_mad_u64_u32 %0, %1, %2, %3, %0\n"
      "v_mad_u64_u32 %0, %1, %4, %5, %0\n"
      "v_mad_u64_u32 %0, %1, %6, %7, %0\n"
      "v_mad_u64_u32 %0, %1, %8, %9, %0\n"
      "v_mad_u64_u32 %0, %1, %10, %11, %0\n"
      "v_mad_u64_u32 %0, %1, %12, %13, %0\n"
      "v_mad_u64_u32 %0, %1, %14, %15, %0\n"
      "v_mad_u64_u32 %0, %1, %16, %17, %0\n"
      "v_mad_u64_u32 %0, %1, %18, %19, %0\n"
      : "+v"(acc), "=&s"(c)
      : "v"(x0), "s"(y0), "v"(x1), "s"(y1), "v"(x2), "s"(y2), "v"(x3), "s"(y3), "v"(x4), "s"(y4), "v"(x5), "s"(y5), "v"(x6), "s"(y6), "v"(x7), "s"(y7), "v"(x8), "s"(y8));
}

// acc += sum_{t < N} x[t] y[t] (both in VGPRs), blocks of at most 18.
template <int N>
__device__ __forceinline__ void mad_vv(uint64_t& acc, const uint32_t* x, const uint32_t* y) {
  if constexpr (N > 18) {
    mad_vv<18>(acc, x, y);
    mad_vv<N - 18>(acc, x + 18, y + 18);
  }
  else if constexpr (N == 1)
    mad_vv1(acc, x[0], y[0]);
  else if constexpr (N == 2)
    mad_vv2(acc, x[0], y[0], x[1], y[1]);
  else if constexpr (N == 3)
    mad_vv3(acc, x[0], y[0], x[1], y[1], x[2], y[2]);
  else if constexpr (N == 4)
    mad_vv4(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3]);
  else if constexpr (N == 5)
    mad_vv5(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4]);
  else if constexpr (N == 6)
    mad_vv6(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5]);
  else if constexpr (N == 7)
    mad_vv7(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6]);
  else if constexpr (N == 8)
    mad_vv8(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7]);
  else if constexpr (N == 9)
    mad_vv9(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8]);
  else if constexpr (N == 10)
    mad_vv10(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8], x[9], y[9]);
  else if constexpr (N == 11)
    mad_vv11(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8], x[9], y[9], x[10], y[10]);
  else if constexpr (N == 12)
    mad_vv12(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8], x[9], y[9], x[10], y[10], x[11], y[11]);
  else if constexpr (N == 13)
    mad_vv13(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8], x[9], y[9], x[10], y[10], x[11], y[11], x[12], y[12]);
  else if constexpr (N == 14)
    mad_vv14(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8], x[9], y[9], x[10], y[10], x[11], y[11], x[12], y[12], x[13], y[13]);
  else if constexpr (N == 15)
    mad_vv15(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8], x[9], y[9], x[10], y[10], x[11], y[11], x[12], y[12], x[13], y[13], x[14], y[14]);
  else if constexpr (N == 16)
    mad_vv16(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8], x[9], y[9], x[10], y[10], x[11], y[11], x[12], y[12], x[13], y[13], x[14], y[14], x[15], y[15]);
  else if constexpr (N == 17)
    mad_vv17(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8], x[9], y[9], x[10], y[10], x[11], y[11], x[12], y[12], x[13], y[13], x[14], y[14], x[15], y[15], x[16], y[16]);
  else if constexpr (N == 18)
    mad_vv18(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8], x[9], y[9], x[10], y[10], x[11], y[11], x[12], y[12], x[13], y[13], x[14], y[14], x[15], y[15], x[16], y[16], x[17], y[17]);
}

// acc += sum_{t < N} x[t] y[t] (y uniform), blocks of at most 9.
template <int N>
__device__ __forceinline__ void mad_vs(uint64_t& acc, const uint32_t* x, const uint32_t* y) {
  if constexpr (N > 9) {
    mad_vs<9>(acc, x, y);
    mad_vs<N - 9>(acc, x + 9, y + 9);
  }
  else if constexpr (N == 1)
    mad_vs1(acc, x[0], y[0]);
  else if constexpr (N == 2)
    mad_vs2(acc, x[0], y[0], x[1], y[1]);
  else if constexpr (N == 3)
    mad_vs3(acc, x[0], y[0], x[1], y[1], x[2], y[2]);
  else if constexpr (N == 4)
    mad_vs4(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3]);
  else if constexpr (N == 5)
    mad_vs5(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4]);
  else if constexpr (N == 6)
    mad_vs6(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5]);
  else if constexpr (N == 7)
    mad_vs7(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6]);
  else if constexpr (N == 8)
    mad_vs8(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7]);
  else if constexpr (N == 9)
    mad_vs9(acc, x[0], y[0], x[1], y[1], x[2], y[2], x[3], y[3], x[4], y[4], x[5], y[5], x[6], y[6], x[7], y[7], x[8], y[8]);
}

}  // namespace zk
