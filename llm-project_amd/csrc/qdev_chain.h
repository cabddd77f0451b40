// qdev_chain.h - the serial add chain of a product-tile pipeline (the decode PV
// kernel's, k_attn.hip).
//
// Layout: three LDS buffers of kChainBufBytes, each 16 rows
// (one per chain) of 128 products plus 4 floats of padding; tile k sits in
// buffer k % 3.  The chain lane of row c adds its 128 products of a tile in
// order, and an s_barrier separates consecutive tiles: with the producers'
// barriers this is the protocol "barrier k certifies that tiles <= k+1 are in
// LDS and that the chains are done with tile k-1".
#ifndef QDEV_CHAIN_H
#define QDEV_CHAIN_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qd {

constexpr int kChainBufBytes = 0x2100;        // 16 rows x (128 + 4) floats

// The chain loop of wave 0 (lane c < kChains owns chain c): for each of the n
// tiles (buffers 0, 1, 2, 0, ... of 0x2100 bytes, rows of kTS floats), 32
// 16-byte LDS reads of the lane's row in four groups of eight, each group
// requested before the previous one is added (s_waitcnt lgkmcnt(8)), the 128
// dependent adds in position order, and the barrier that ends the tile (not
// after the last one).  The first group of the next tile is requested before
// that barrier: the tile has been in LDS since the previous barrier.
// Written as one asm block because the reads run with exec = lanes 0-15 (one
// wave's 64-lane 16-byte LDS read costs it about 40 clocks of issue, the
// 16-lane one about a quarter of that) and the compiler would otherwise copy the
// conditionally read registers and wait for every read before the adds.  Lanes
// 16-63 add whatever their registers hold; their sums are never stored.  Every
// read has landed when the block ends (lgkmcnt(0)), so that no late return
// writes a register the compiler reuses.
#define PV_RA(o0, o1, o2, o3, o4, o5, o6, o7)                                                              \
  "ds_read_b128 v[100:103], %[ad] offset:" #o0 "\n\t"                                                     \
  "ds_read_b128 v[104:107], %[ad] offset:" #o1 "\n\t"                                                     \
  "ds_read_b128 v[108:111], %[ad] offset:" #o2 "\n\t"                                                     \
  "ds_read_b128 v[112:115], %[ad] offset:" #o3 "\n\t"                                                     \
  "ds_read_b128 v[116:119], %[ad] offset:" #o4 "\n\t"                                                     \
  "ds_read_b128 v[120:123], %[ad] offset:" #o5 "\n\t"                                                     \
  "ds_read_b128 v[124:127], %[ad] offset:" #o6 "\n\t"                                                     \
  "ds_read_b128 v[128:131], %[ad] offset:" #o7 "\n\t"
#define PV_RB(o0, o1, o2, o3, o4, o5, o6, o7)                                                              \
  "ds_read_b128 v[132:135], %[ad] offset:" #o0 "\n\t"                                                     \
  "ds_read_b128 v[136:139], %[ad] offset:" #o1 "\n\t"                                                     \
  "ds_read_b128 v[140:143], %[ad] offset:" #o2 "\n\t"                                                     \
  "ds_read_b128 v[144:147], %[ad] offset:" #o3 "\n\t"                                                     \
  "ds_read_b128 v[148:151], %[ad] offset:" #o4 "\n\t"                                                     \
  "ds_read_b128 v[152:155], %[ad] offset:" #o5 "\n\t"                                                     \
  "ds_read_b128 v[156:159], %[ad] offset:" #o6 "\n\t"                                                     \
  "ds_read_b128 v[160:163], %[ad] offset:" #o7 "\n\t"
#define PV_X16(reads) "s_mov_b64 %[sx], exec\n\ts_mov_b64 exec, 0xffff\n\t" reads "s_mov_b64 exec, %[sx]\n\t"
#define PV_A1(r) "v_add_f32 %[acc], %[acc], v" #r "\n\t"
#define PV_A4(a, b, c, d) PV_A1(a) PV_A1(b) PV_A1(c) PV_A1(d)
#define PV_ADD_A                                                                                           \
  PV_A4(100, 101, 102, 103) PV_A4(104, 105, 106, 107) PV_A4(108, 109, 110, 111) PV_A4(112, 113, 114, 115)  \
  PV_A4(116, 117, 118, 119) PV_A4(120, 121, 122, 123) PV_A4(124, 125, 126, 127) PV_A4(128, 129, 130, 131)
#define PV_ADD_B                                                                                           \
  PV_A4(132, 133, 134, 135) PV_A4(136, 137, 138, 139) PV_A4(140, 141, 142, 143) PV_A4(144, 145, 146, 147)  \
  PV_A4(148, 149, 150, 151) PV_A4(152, 153, 154, 155) PV_A4(156, 157, 158, 159) PV_A4(160, 161, 162, 163)

__device__ __forceinline__ void chain_tiles_asm(float &acc, unsigned base, int n) {
  unsigned ad, bo;
  uint64_t sx;
  asm volatile(
      "s_waitcnt lgkmcnt(0)\n\t"
      "s_mov_b32 %[bo], 0\n\t"
      "v_mov_b32 %[ad], %[base]\n\t"
      PV_X16(PV_RA(0, 16, 32, 48, 64, 80, 96, 112))
      "1:\n\t"
      PV_X16(PV_RB(128, 144, 160, 176, 192, 208, 224, 240))
      "s_waitcnt lgkmcnt(8)\n\t" PV_ADD_A
      PV_X16(PV_RA(256, 272, 288, 304, 320, 336, 352, 368))
      "s_waitcnt lgkmcnt(8)\n\t" PV_ADD_B
      PV_X16(PV_RB(384, 400, 416, 432, 448, 464, 480, 496))
      "s_waitcnt lgkmcnt(8)\n\t" PV_ADD_A
      "s_add_u32 %[bo], %[bo], 0x2100\n\t"
      "s_cmp_eq_u32 %[bo], 0x6300\n\t"
      "s_cselect_b32 %[bo], 0, %[bo]\n\t"
      "v_add_u32 %[ad], %[bo], %[base]\n\t"
      PV_X16(PV_RA(0, 16, 32, 48, 64, 80, 96, 112))
      "s_waitcnt lgkmcnt(8)\n\t" PV_ADD_B
      "s_sub_u32 %[n], %[n], 1\n\t"
      "s_cmp_eq_u32 %[n], 0\n\t"
      "s_cbranch_scc1 2f\n\t"
      "s_waitcnt lgkmcnt(0)\n\t"
      "s_barrier\n\t"
      "s_branch 1b\n"
      "2:\n\t"
      "s_waitcnt lgkmcnt(0)"
      : [acc] "+v"(acc), [ad] "=&v"(ad), [bo] "=&s"(bo), [n] "+s"(n), [sx] "=&s"(sx)
      : [base] "v"(base)
      : "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111", "v112",
        "v113", "v114", "v115", "v116", "v117", "v118", "v119", "v120", "v121", "v122", "v123", "v124", "v125",
        "v126", "v127", "v128", "v129", "v130", "v131", "v132", "v133", "v134", "v135", "v136", "v137", "v138",
        "v139", "v140", "v141", "v142", "v143", "v144", "v145", "v146", "v147", "v148", "v149", "v150", "v151",
        "v152", "v153", "v154", "v155", "v156", "v157", "v158", "v159", "v160", "v161", "v162", "v163", "scc",
        "memory");
}
#undef PV_RA
#undef PV_RB
#undef PV_X16
#undef PV_A1
#undef PV_A4
#undef PV_ADD_A
#undef PV_ADD_B

}  // namespace qd

#endif
