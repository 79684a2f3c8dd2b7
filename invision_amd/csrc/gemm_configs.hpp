// gemm_configs.hpp -- the instantiated GEMM tile configurations.
//
// INV_CFG_<id> is the configuration type:
//  inv::TileCfg<TN, TM, WN, WM, BK, NST>: a TN x TM output tile (W rows x X
//    rows), WN x WM waves of 64 threads, BK-wide k-tiles, NST-stage LDS ring
//    filled by direct global->LDS copies;
//  inv::RsCfg<TN, TM, WN, WM, NREG, PF>: 64-wide k-tiles, two LDS buffers
//    filled from NREG register stages of global prefetch, MFMA fragments read
//    PF 16-wide substeps ahead;
//  inv::Rs16Cfg<TN, TM, WN, WM, NREG>: the same on 16x16x32 MFMAs (16-row
//    blocks), fragments one 32-wide substep ahead.
// Each configuration is compiled in its own translation unit
// (gemm_instance.hip with -DINV_CFG_ID=<id>) and reached through
// inv_gemm_launch_<id>.  The types are defined in gemm_kernel.hpp.
#pragma once

#include <hip/hip_runtime.h>

#define INV_CFG_0 inv::TileCfg<256, 256, 2, 4, 32, 4> /* 8 waves of 128x64, 4-stage ring (128 KiB) */
#define INV_CFG_1 inv::TileCfg<256, 256, 2, 4, 32, 5> /* same, 5 stages (160 KiB) */
#define INV_CFG_2 inv::TileCfg<256, 128, 2, 2, 64, 3> /* 4 waves of 128x64 */
#define INV_CFG_3 inv::TileCfg<128, 128, 2, 2, 64, 4> /* 4 waves of 64x64 */
#define INV_CFG_4 inv::TileCfg<128, 64, 2, 2, 64, 4> /* 4 waves of 64x32 */
#define INV_CFG_5 inv::TileCfg<128, 32, 4, 1, 64, 4> /* 4 waves of 32x32: W streaming for M <= 32 */
#define INV_CFG_6 inv::TileCfg<256, 256, 4, 2, 32, 4> /* 8 waves of 64x128 */
#define INV_CFG_7 inv::TileCfg<256, 256, 2, 2, 32, 4> /* 4 waves of 128x128 */

#define INV_CFG_8 inv::RsCfg<256, 256, 2, 2, 2> /* 4 waves of 128x128, two register stages */
#define INV_CFG_9 inv::RsCfg<256, 256, 2, 2, 1> /* same, one register stage */
#define INV_CFG_10 inv::RsCfg<256, 256, 2, 2, 1, 2> /* one register stage, fragments two substeps ahead */
#define INV_CFG_11 inv::RsCfg<256, 224, 4, 1, 2> /* 4 waves of 64x224 (W rows x X rows) */
#define INV_CFG_12 inv::RsCfg<224, 256, 1, 4, 2> /* 4 waves of 224x64 */
#define INV_CFG_13 inv::RsCfg<256, 128, 2, 2, 2> /* 4 waves of 128x64: half-height X tile */
#define INV_CFG_14 inv::RsCfg<128, 256, 2, 2, 2> /* 4 waves of 64x128: half-height W tile */
#define INV_CFG_15 inv::RsCfg<128, 128, 2, 2, 2> /* 4 waves of 64x64: small problems, two workgroups per CU */

#define INV_CFG_16 inv::Rs16Cfg<256, 224, 2, 2, 1> /* 16x16x32 MFMAs, 4 waves of 128x112, one register stage */
#define INV_CFG_17 inv::Rs16Cfg<256, 256, 2, 4, 1> /* 16x16x32 MFMAs, 8 waves of 128x64, two per SIMD */
#define INV_CFG_18 inv::Rs16Cfg<256, 192, 2, 2, 1> /* 16x16x32 MFMAs, 4 waves of 128x96, one register stage */

#define INV_GEMM_CONFIG_IDS(X) \
    X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(15) X(16) X(17) X(18)
#define INV_GEMM_NUM_CONFIGS 19

namespace inv {
struct GemmParams;
}

#define INV_DECLARE_LAUNCH(id) \
    hipError_t inv_gemm_launch_##id(const inv::GemmParams &p, int epi, int out, int mode, hipStream_t s);
INV_GEMM_CONFIG_IDS(INV_DECLARE_LAUNCH)
#undef INV_DECLARE_LAUNCH
