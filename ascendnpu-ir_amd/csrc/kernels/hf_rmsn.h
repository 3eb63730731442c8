// RMSNorm + dynamic per-row int8 quantisation with the reference's serial
// sum (the default kernel for the pattern; lower.cpp matchRmsQuant).
//
// The group (compile-rms-norm-fp32-split-n.mlir:5-47 followed by the
// quantisation of the configs): ss = serial fold from s0 of RN(x_c^2);
// inv = rec(sqrt(ss / K + eps)); y_c = RN(RN(x_c * inv) * g_c);
// amax = maximumf(a0, max_c |y_c|); sc = RN(amax / QD);
// q_c = int8(maxf(minf(rint(RN(y_c / sc)), HI), LO)).
//
// The int8 codes depend on the exact serial sum, so each row's 4096 squares
// are added in column order by one lane: a latency-bound chain of C dependent
// adds.  The block is laid out around it:
//  - 32 rows per block, 9 waves: wave 0 only runs the chains (lanes 0..31,
//    one row each); waves 1..8 hold 4 rows each as packed bf16 in registers
//    (lane l owns columns 512 j + 8 l .. +7 of every 512-column chunk j).
//    Three waves per SIMD leave 168 VGPRs a wave: 128 hold the rows.
//  - Round k: the row waves write the f32 squares of chunk k into one of two
//    LDS slots (32 rows x 516 floats), a barrier publishes it, and the chain
//    wave folds it while the row waves write chunk k+1.  Loads run two chunks
//    ahead of the chain.
//  - While the chain runs, the row waves also reduce the exact products
//    p_c = |x_c * g_c| (bf16 x bf16 is exact in f32) to a per-lane maximum
//    and the set of chunks holding it.  y_c is within 2^-23 relative of
//    p_c * inv and distinct products differ by at least 2^-16 relative, so
//    max |y| is attained where p is maximal; after the chain only the chunks
//    of the lanes holding the row's maximal p recompute y for amax.
//    The argument needs the products near the maximum and their y far from
//    underflow (p >= 2^-100, p * inv >= 2^-90: the rounding errors are then
//    relative); a zero row, a non-normal reciprocal or scale, a non-finite
//    gamma or a quant8x4 guard sends the block to a plain serial
//    re-execution (rmsn_exact).
//  - The tail quantises from registers (hf::quant8x4), four codes at a time.
#pragma once
#include "hf_ops.h"
#include "hf_rmsq.h" // wave_max

namespace hf {

// Lanes of the chain wave fold the 512 floats at rp (one row's chunk) into
// acc in order: 32 groups of 16 floats through two register buffers
// (v128-v159), the reads of group g+2 in flight while group g is added.
__device__ __forceinline__ float rmsn_chain512(const float *rp, float acc) {
  const uint32_t p = (uint32_t)(uintptr_t)rp;
  asm volatile(
      "ds_read_b128 v[128:131], %[p] offset:0\n" "ds_read_b128 v[132:135], %[p] offset:16\n" "ds_read_b128 v[136:139], %[p] offset:32\n" "ds_read_b128 v[140:143], %[p] offset:48\n" "ds_read_b128 v[144:147], %[p] offset:64\n" "ds_read_b128 v[148:151], %[p] offset:80\n" "ds_read_b128 v[152:155], %[p] offset:96\n" "ds_read_b128 v[156:159], %[p] offset:112\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:128\n" "ds_read_b128 v[132:135], %[p] offset:144\n" "ds_read_b128 v[136:139], %[p] offset:160\n" "ds_read_b128 v[140:143], %[p] offset:176\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:192\n" "ds_read_b128 v[148:151], %[p] offset:208\n" "ds_read_b128 v[152:155], %[p] offset:224\n" "ds_read_b128 v[156:159], %[p] offset:240\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:256\n" "ds_read_b128 v[132:135], %[p] offset:272\n" "ds_read_b128 v[136:139], %[p] offset:288\n" "ds_read_b128 v[140:143], %[p] offset:304\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:320\n" "ds_read_b128 v[148:151], %[p] offset:336\n" "ds_read_b128 v[152:155], %[p] offset:352\n" "ds_read_b128 v[156:159], %[p] offset:368\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:384\n" "ds_read_b128 v[132:135], %[p] offset:400\n" "ds_read_b128 v[136:139], %[p] offset:416\n" "ds_read_b128 v[140:143], %[p] offset:432\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:448\n" "ds_read_b128 v[148:151], %[p] offset:464\n" "ds_read_b128 v[152:155], %[p] offset:480\n" "ds_read_b128 v[156:159], %[p] offset:496\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:512\n" "ds_read_b128 v[132:135], %[p] offset:528\n" "ds_read_b128 v[136:139], %[p] offset:544\n" "ds_read_b128 v[140:143], %[p] offset:560\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:576\n" "ds_read_b128 v[148:151], %[p] offset:592\n" "ds_read_b128 v[152:155], %[p] offset:608\n" "ds_read_b128 v[156:159], %[p] offset:624\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:640\n" "ds_read_b128 v[132:135], %[p] offset:656\n" "ds_read_b128 v[136:139], %[p] offset:672\n" "ds_read_b128 v[140:143], %[p] offset:688\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:704\n" "ds_read_b128 v[148:151], %[p] offset:720\n" "ds_read_b128 v[152:155], %[p] offset:736\n" "ds_read_b128 v[156:159], %[p] offset:752\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:768\n" "ds_read_b128 v[132:135], %[p] offset:784\n" "ds_read_b128 v[136:139], %[p] offset:800\n" "ds_read_b128 v[140:143], %[p] offset:816\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:832\n" "ds_read_b128 v[148:151], %[p] offset:848\n" "ds_read_b128 v[152:155], %[p] offset:864\n" "ds_read_b128 v[156:159], %[p] offset:880\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:896\n" "ds_read_b128 v[132:135], %[p] offset:912\n" "ds_read_b128 v[136:139], %[p] offset:928\n" "ds_read_b128 v[140:143], %[p] offset:944\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:960\n" "ds_read_b128 v[148:151], %[p] offset:976\n" "ds_read_b128 v[152:155], %[p] offset:992\n" "ds_read_b128 v[156:159], %[p] offset:1008\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:1024\n" "ds_read_b128 v[132:135], %[p] offset:1040\n" "ds_read_b128 v[136:139], %[p] offset:1056\n" "ds_read_b128 v[140:143], %[p] offset:1072\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:1088\n" "ds_read_b128 v[148:151], %[p] offset:1104\n" "ds_read_b128 v[152:155], %[p] offset:1120\n" "ds_read_b128 v[156:159], %[p] offset:1136\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:1152\n" "ds_read_b128 v[132:135], %[p] offset:1168\n" "ds_read_b128 v[136:139], %[p] offset:1184\n" "ds_read_b128 v[140:143], %[p] offset:1200\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:1216\n" "ds_read_b128 v[148:151], %[p] offset:1232\n" "ds_read_b128 v[152:155], %[p] offset:1248\n" "ds_read_b128 v[156:159], %[p] offset:1264\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:1280\n" "ds_read_b128 v[132:135], %[p] offset:1296\n" "ds_read_b128 v[136:139], %[p] offset:1312\n" "ds_read_b128 v[140:143], %[p] offset:1328\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:1344\n" "ds_read_b128 v[148:151], %[p] offset:1360\n" "ds_read_b128 v[152:155], %[p] offset:1376\n" "ds_read_b128 v[156:159], %[p] offset:1392\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:1408\n" "ds_read_b128 v[132:135], %[p] offset:1424\n" "ds_read_b128 v[136:139], %[p] offset:1440\n" "ds_read_b128 v[140:143], %[p] offset:1456\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:1472\n" "ds_read_b128 v[148:151], %[p] offset:1488\n" "ds_read_b128 v[152:155], %[p] offset:1504\n" "ds_read_b128 v[156:159], %[p] offset:1520\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:1536\n" "ds_read_b128 v[132:135], %[p] offset:1552\n" "ds_read_b128 v[136:139], %[p] offset:1568\n" "ds_read_b128 v[140:143], %[p] offset:1584\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:1600\n" "ds_read_b128 v[148:151], %[p] offset:1616\n" "ds_read_b128 v[152:155], %[p] offset:1632\n" "ds_read_b128 v[156:159], %[p] offset:1648\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:1664\n" "ds_read_b128 v[132:135], %[p] offset:1680\n" "ds_read_b128 v[136:139], %[p] offset:1696\n" "ds_read_b128 v[140:143], %[p] offset:1712\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:1728\n" "ds_read_b128 v[148:151], %[p] offset:1744\n" "ds_read_b128 v[152:155], %[p] offset:1760\n" "ds_read_b128 v[156:159], %[p] offset:1776\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:1792\n" "ds_read_b128 v[132:135], %[p] offset:1808\n" "ds_read_b128 v[136:139], %[p] offset:1824\n" "ds_read_b128 v[140:143], %[p] offset:1840\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:1856\n" "ds_read_b128 v[148:151], %[p] offset:1872\n" "ds_read_b128 v[152:155], %[p] offset:1888\n" "ds_read_b128 v[156:159], %[p] offset:1904\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" "ds_read_b128 v[128:131], %[p] offset:1920\n" "ds_read_b128 v[132:135], %[p] offset:1936\n" "ds_read_b128 v[136:139], %[p] offset:1952\n" "ds_read_b128 v[140:143], %[p] offset:1968\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" "ds_read_b128 v[144:147], %[p] offset:1984\n" "ds_read_b128 v[148:151], %[p] offset:2000\n" "ds_read_b128 v[152:155], %[p] offset:2016\n" "ds_read_b128 v[156:159], %[p] offset:2032\n" 
      "s_waitcnt lgkmcnt(4)\n" "v_add_f32 %[acc], v128, %[acc]\n" "v_add_f32 %[acc], v129, %[acc]\n" "v_add_f32 %[acc], v130, %[acc]\n" "v_add_f32 %[acc], v131, %[acc]\n" "v_add_f32 %[acc], v132, %[acc]\n" "v_add_f32 %[acc], v133, %[acc]\n" "v_add_f32 %[acc], v134, %[acc]\n" "v_add_f32 %[acc], v135, %[acc]\n" "v_add_f32 %[acc], v136, %[acc]\n" "v_add_f32 %[acc], v137, %[acc]\n" "v_add_f32 %[acc], v138, %[acc]\n" "v_add_f32 %[acc], v139, %[acc]\n" "v_add_f32 %[acc], v140, %[acc]\n" "v_add_f32 %[acc], v141, %[acc]\n" "v_add_f32 %[acc], v142, %[acc]\n" "v_add_f32 %[acc], v143, %[acc]\n" 
      "s_waitcnt lgkmcnt(0)\n" "v_add_f32 %[acc], v144, %[acc]\n" "v_add_f32 %[acc], v145, %[acc]\n" "v_add_f32 %[acc], v146, %[acc]\n" "v_add_f32 %[acc], v147, %[acc]\n" "v_add_f32 %[acc], v148, %[acc]\n" "v_add_f32 %[acc], v149, %[acc]\n" "v_add_f32 %[acc], v150, %[acc]\n" "v_add_f32 %[acc], v151, %[acc]\n" "v_add_f32 %[acc], v152, %[acc]\n" "v_add_f32 %[acc], v153, %[acc]\n" "v_add_f32 %[acc], v154, %[acc]\n" "v_add_f32 %[acc], v155, %[acc]\n" "v_add_f32 %[acc], v156, %[acc]\n" "v_add_f32 %[acc], v157, %[acc]\n" "v_add_f32 %[acc], v158, %[acc]\n" "v_add_f32 %[acc], v159, %[acc]\n" 
      : [acc] "+v"(acc) : [p] "v"(p)
      : "v128", "v129", "v130", "v131", "v132", "v133", "v134", "v135", "v136", "v137", "v138", "v139", "v140", "v141", "v142", "v143", "v144", "v145", "v146", "v147", "v148", "v149", "v150", "v151", "v152", "v153", "v154", "v155", "v156", "v157", "v158", "v159", "memory");

  return acc;
}

// a wave-uniform value, kept in an SGPR
__device__ __forceinline__ float uniform(float v) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))); }

// forget what the compiler knows about the resident words (so it recomputes
// unpacked values instead of keeping them alive across phases)
template <int N>
__device__ __forceinline__ void launder_words(uint4 (&a)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(a[i].x), "+v"(a[i].y), "+v"(a[i].z), "+v"(a[i].w));
}

__device__ __forceinline__ void unpack8(const uint4 &v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = u2f(w[i] << 16);
    f[2 * i + 1] = u2f(w[i] & 0xFFFF0000u);
  }
}

constexpr int RMSN_ROWS = 32, RMSN_STRIDE = 516, RMSN_THREADS = 576;

// Plain re-execution of the block's rows: one lane per row for the serial
// sums, then one wave per row for amax and the codes, every operation as the
// group states it (IEEE division).
template <int C, int LO, int HI>
__device__ __attribute__((noinline)) void rmsn_exact(const uint16_t *__restrict__ x, const uint16_t *__restrict__ gamma,
                                                      int8_t *__restrict__ q, float *__restrict__ scale, int64_t R,
                                                      float s0, float K, float eps, float a0, float qd, float *sh) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t row0 = (int64_t)blockIdx.x * RMSN_ROWS;
  __syncthreads();
  if (tid < RMSN_ROWS) {
    const int64_t r = row0 + tid < R ? row0 + tid : R - 1;
    float ss = s0;
    for (int c = 0; c < C; ++c) {
      const float xf = bf16_to_f32(x[r * C + c]);
      ss = ss + xf * xf;
    }
    sh[tid] = rec(__builtin_sqrtf(ss / K + eps));
  }
  __syncthreads();
  for (int rl = wave; rl < RMSN_ROWS; rl += RMSN_THREADS / 64) {
    const int64_t r = row0 + rl < R ? row0 + rl : R - 1;
    const float inv = sh[rl];
    float m = -__builtin_inff();
    for (int c = lane; c < C; c += 64) {
      const float y = (bf16_to_f32(x[r * C + c]) * inv) * bf16_to_f32(gamma[c]);
      m = maximumf(__builtin_fabsf(y), m);
    }
    const float amax = maximumf(wave_max(m), a0);
    const float sc = amax / qd;
    if (lane == 0 && row0 + rl < R) scale[r] = sc;
    for (int c = lane; c < C; c += 64) {
      const float y = (bf16_to_f32(x[r * C + c]) * inv) * bf16_to_f32(gamma[c]);
      float v = __builtin_roundevenf(y / sc);
      v = maximumf(minimumf(v, (float)HI), (float)LO);
      q[r * C + c] = (int8_t)(int32_t)v;
    }
  }
}

// NaN-propagating maximum over the 64 lanes of N values at once (the DPP
// steps of the N reductions interleaved), returned wave-uniform
template <int N>
__device__ __forceinline__ void wave_max_n(float (&v)[N]) {
#define HF_STEP(...)                                                                                       \
  _Pragma("unroll") for (int i = 0; i < N; ++i) v[i] =                                                     \
      maximumf(v[i], __int_as_float(dpp<__VA_ARGS__>(__float_as_int(v[i]), __float_as_int(v[i]))));
  HF_STEP(DPP_ROW_SHR1)
  HF_STEP(DPP_ROW_SHR2)
  HF_STEP(DPP_ROW_SHR4)
  HF_STEP(DPP_ROW_SHR8)
  HF_STEP(DPP_ROW_BCAST15, 0xa)
  HF_STEP(DPP_ROW_BCAST31, 0xc)
#undef HF_STEP
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[i]), 63));
}

// The chain wave: for each chunk, wait for the barrier that publishes it,
// then fold it (lanes 0..31, one row each); the sums go to sh.
template <int NCH>
__device__ __forceinline__ bool rmsn_chain_wave(const float *ring, float *sh, float s0, int lane) {
  // the chain is the block's critical path: its wave issues first on its SIMD
  __builtin_amdgcn_s_setprio(3);
  float acc = s0;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    __syncthreads(); // chunk k published
    if (lane < RMSN_ROWS) acc = rmsn_chain512(ring + (k & 1) * RMSN_ROWS * RMSN_STRIDE + lane * RMSN_STRIDE, acc);
  }
  if (lane < RMSN_ROWS) sh[lane] = acc;
  __syncthreads(); // sums published
  return __syncthreads_or(0);
}

// A row wave: block rows rbase .. rbase + RPW - 1.
template <int C, int LO, int HI, int RPW>
__device__ __forceinline__ bool rmsn_row_wave(const uint16_t *__restrict__ x, const uint16_t *__restrict__ gamma,
                                              int8_t *__restrict__ q, float *__restrict__ scale, int64_t R, float K,
                                              float eps, float a0, float qd, float *ring, uint16_t *g_lds,
                                              const float *sh, int w, int rbase, int lane) {
  constexpr int NCH = C / 512;
  const int64_t row0 = (int64_t)blockIdx.x * RMSN_ROWS;
  int64_t grow[RPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int64_t r = row0 + rbase + rr;
    grow[rr] = r < R ? r : R - 1;
  }
  bool bad = false;
  // gamma first (8 KB, shared by every block: mostly L2 hits), so that its
  // LDS copy does not wait behind the rows' loads
  uint4 gv = make_uint4(0, 0, 0, 0);
  const int gi = w * 64 + lane;
  if (gi < C / 8) gv = *(const uint4 *)(gamma + gi * 8);
  uint4 xv[RPW][NCH];
  auto issue = [&](int j) {
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) xv[rr][j] = *(const uint4 *)(x + grow[rr] * C + j * 512 + lane * 8);
  };
  issue(0);
#ifndef HF_RMSN_LA0
#define HF_RMSN_LA0 2
#endif
  if (HF_RMSN_LA0 > 1 && NCH > 1) issue(1);
  // the gamma copy is published by the first chunk's barrier; a non-finite
  // gamma takes the exact path
  if (gi < C / 8) {
    *(uint4 *)(g_lds + gi * 8) = gv;
    const uint32_t ww[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) bad |= (ww[k] & 0x7F80u) == 0x7F80u || ((ww[k] >> 16) & 0x7F80u) == 0x7F80u;
  }
  bad = __builtin_amdgcn_ballot_w64(bad) != 0; // wave-uniform: an SGPR pair
  float pmax[RPW];
  uint32_t pmask[RPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) { pmax[rr] = 0.0f; pmask[rr] = 0; }
  // the exact products |x * g| of chunk j reduced to the lane's maximum and
  // the set of chunks holding it (branch-free), computed in place
  auto products = [&](int j) {
    float gf[8];
    unpack8(*(const uint4 *)(g_lds + j * 512 + lane * 8), gf);
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      float xf[8];
      unpack8(xv[rr][j], xf);
      float cm = 0.0f;
#pragma unroll
      for (int v = 0; v < 8; ++v) cm = __builtin_fmaxf(cm, __builtin_fabsf(xf[v] * gf[v]));
      const uint32_t gt = cm > pmax[rr] ? ~0u : 0u, ge = cm >= pmax[rr] ? ~0u : 0u;
      pmask[rr] = (pmask[rr] & ~gt) | ((1u << j) & ge);
      pmax[rr] = __builtin_fmaxf(pmax[rr], cm);
      asm volatile("" : "+v"(pmax[rr]), "+v"(pmask[rr]));
    }
  };
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    // chunk k's squares into its slot (the chain finished the slot's
    // previous chunk before the last barrier); chunk k-1's products (gamma
    // is visible from the first barrier on); loads two chunks ahead
    float *slot = ring + (k & 1) * RMSN_ROWS * RMSN_STRIDE;
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      float xf[8];
      unpack8(xv[rr][k], xf);
      float *dst = slot + (rbase + rr) * RMSN_STRIDE + lane * 8;
      *(float4 *)dst = make_float4(xf[0] * xf[0], xf[1] * xf[1], xf[2] * xf[2], xf[3] * xf[3]);
      *(float4 *)(dst + 4) = make_float4(xf[4] * xf[4], xf[5] * xf[5], xf[6] * xf[6], xf[7] * xf[7]);
      // the unpacked values die here; the products unpack again
      asm volatile("" : "+v"(xv[rr][k].x), "+v"(xv[rr][k].y), "+v"(xv[rr][k].z), "+v"(xv[rr][k].w));
    }
    if (HF_RMSN_LA0 == 1 && k == 0 && NCH > 1) issue(1);
    if (k + 2 < NCH) issue(k + 2);
    if (k >= 1) products(k - 1);
    __syncthreads(); // chunk k published
  }
  products(NCH - 1);
  __syncthreads(); // sums published
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) launder_words(xv[rr]);
  Guard hg;
  // per-row values are wave-uniform (a wave holds whole rows): SGPRs
  float inv[RPW], pm[RPW], am[RPW], sc[RPW], rc[RPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    inv[rr] = uniform(rec(__builtin_sqrtf(sh[rbase + rr] / K + eps)));
    pm[rr] = pmax[rr];
  }
  wave_max_n(pm);
  // amax from the chunks holding the row's maximal product: a chunk is
  // taken (a wave-uniform branch) when some lane whose maximum equals the
  // row's has it in its set, usually one chunk; every lane then folds |y|
  // over its columns of that chunk (a lane whose products are smaller cannot
  // exceed the maximum).  Exact when the products near the maximum and their
  // y stay far from underflow.
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    bad |= !(inv[rr] >= 0x1p-100f && inv[rr] <= 0x1p+100f && pm[rr] >= 0x1p-100f && pm[rr] * inv[rr] >= 0x1p-90f);
    const bool cand = pmax[rr] == pm[rr];
    am[rr] = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
      if (__builtin_amdgcn_ballot_w64(cand && (pmask[rr] >> j & 1u)) != 0) {
        float gf[8], xf[8];
        unpack8(*(const uint4 *)(g_lds + j * 512 + lane * 8), gf);
        unpack8(xv[rr][j], xf);
#pragma unroll
        for (int v = 0; v < 8; ++v) am[rr] = maximumf(am[rr], __builtin_fabsf((xf[v] * inv[rr]) * gf[v]));
      }
  }
  wave_max_n(am);
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    launder_words(xv[rr]);
    sc[rr] = uniform(maximumf(am[rr], a0) / qd);
    rc[rr] = uniform(1.0f / sc[rr]);
    hg.divisor(rc[rr]);
  }
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    // gamma of the chunk once for the wave's rows
    float gf[8];
    unpack8(*(const uint4 *)(g_lds + j * 512 + lane * 8), gf);
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      float xf[8];
      unpack8(xv[rr][j], xf);
      uint2 st;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = (xf[4 * h + i] * inv[rr]) * gf[4 * h + i];
        (h ? st.y : st.x) = quant8x4<LO, HI>(y, sc[rr], rc[rr], hg);
      }
      *(uint2 *)(q + grow[rr] * C + j * 512 + lane * 8) = st;
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (lane == 0)
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr)
      if (row0 + rbase + rr < R) scale[grow[rr]] = sc[rr];
  bad |= hg.bad();
  return __syncthreads_or(bad);
}

// The block: wave 0 runs the chains, waves 1..8 the rows.  Both kinds of
// wave meet at the same barriers (the same count, in order); the branch is
// wave-uniform.
template <int C, int LO, int HI>
__device__ __forceinline__ void rmsn_rows(const uint16_t *__restrict__ x, const uint16_t *__restrict__ gamma,
                                          int8_t *__restrict__ q, float *__restrict__ scale, int64_t R, float s0, float K,
                                          float eps, float a0, float qd) {
  static_assert(C % 512 == 0 && C >= 512 && C <= 4096, "rows of 512 to 4096 columns in 512-column chunks");
  __shared__ __attribute__((aligned(16))) float ring[2 * RMSN_ROWS * RMSN_STRIDE];
  __shared__ __attribute__((aligned(16))) uint16_t g_lds[C];
  __shared__ float sh[RMSN_ROWS];
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
  bool bad;
  if (wave == 0) {
    bad = rmsn_chain_wave<C / 512>(ring, sh, s0, lane);
  } else {
    // waves 1..4: five rows each, waves 5..7: four
    const int w = wave - 1;
    bad = rmsn_row_wave<C, LO, HI, 4>(x, gamma, q, scale, R, K, eps, a0, qd, ring, g_lds, sh, w, 4 * w, lane);
  }
  if (bad) rmsn_exact<C, LO, HI>(x, gamma, q, scale, R, s0, K, eps, a0, qd, sh);
}

} // namespace hf
