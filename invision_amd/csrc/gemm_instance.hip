// gemm_instance.hip -- one translation unit per tile configuration: compiled
// with -DINV_CFG_ID=<id>, it instantiates gemm_nt_bf16_kernel for that
// configuration's epilogues, output types and split-K modes and defines
// inv_gemm_launch_<id>.
#include "gemm_configs.hpp"
#include "gemm_kernel.hpp"

#ifndef INV_CFG_ID
#error "compile with -DINV_CFG_ID=<configuration id>"
#endif

namespace {

template <class C, int EPI, int OUT, int MODE, bool GATHER = false>
void launch_one(const inv::GemmParams &p, dim3 grid, dim3 block, hipStream_t s) {
    hipLaunchKernelGGL((inv::gemm_nt_bf16_kernel<C, EPI, OUT, MODE, GATHER>), grid, block, 0, s, p);
}

// Tile configurations with the implicit-convolution (gather) instantiation:
// 256x256 (one register stage: the gather offsets and tap masks take the
// registers of the second) and 256x224 for many output channels, 256x128 for
// 128 or fewer.
constexpr bool kGatherCfg = INV_CFG_ID == 9 || INV_CFG_ID == 13 || INV_CFG_ID == 16;

template <class C, int MODE>
bool launch_epi(const inv::GemmParams &p, int epi, int out, dim3 grid, dim3 block, hipStream_t s) {
    const bool f32 = out == inv::OUT_F32;
    if (epi == inv::EPI_SILU) {
        if (f32) launch_one<C, inv::EPI_SILU, inv::OUT_F32, MODE>(p, grid, block, s);
        else launch_one<C, inv::EPI_SILU, inv::OUT_BF16, MODE>(p, grid, block, s);
    } else if (epi == inv::EPI_GELU) {
        if (f32) launch_one<C, inv::EPI_GELU, inv::OUT_F32, MODE>(p, grid, block, s);
        else launch_one<C, inv::EPI_GELU, inv::OUT_BF16, MODE>(p, grid, block, s);
    } else if (epi == inv::EPI_ROWBIAS) {
        if constexpr (C::STAGED_EPI) {
            if (f32) launch_one<C, inv::EPI_ROWBIAS, inv::OUT_F32, MODE>(p, grid, block, s);
            else launch_one<C, inv::EPI_ROWBIAS, inv::OUT_BF16, MODE>(p, grid, block, s);
            return true;
        }
        return false;
    } else if (epi == inv::EPI_SWIGLU) {
        // only one workgroup per tile, and only where the tile splits into gate | up wave columns
        if constexpr (C::SWIGLU_OK && MODE == inv::GRID_TILES) {
            if (f32) launch_one<C, inv::EPI_SWIGLU, inv::OUT_F32, MODE>(p, grid, block, s);
            else launch_one<C, inv::EPI_SWIGLU, inv::OUT_BF16, MODE>(p, grid, block, s);
            return true;
        }
        return false;
    } else {
        if (f32) launch_one<C, inv::EPI_NONE, inv::OUT_F32, MODE>(p, grid, block, s);
        else launch_one<C, inv::EPI_NONE, inv::OUT_BF16, MODE>(p, grid, block, s);
    }
    return true;
}

// mode: inv::GRID_TILES (one workgroup per tile), GRID_SPLITK (tiles x ksplit
// workgroups) or GRID_STREAMK (p.ksplit is then the persistent grid size).
template <class C>
hipError_t launch_cfg(const inv::GemmParams &p, int epi, int out, int mode, hipStream_t s) {
    dim3 block(C::NTHREADS);
    // tiles of this launch: p.tile_count from p.tile_base, or all of them
    const unsigned ntiles = (unsigned)(p.tile_count > 0 ? p.tile_count : p.tiles_m * p.tiles_n);
    bool ok;
    if (mode == inv::LAUNCH_GATHER) {
        if constexpr (kGatherCfg && C::REG_STAGED && C::STAGED_EPI) {
            if (epi != inv::EPI_ROWBIAS || out != inv::OUT_F32) return hipErrorInvalidConfiguration;
            launch_one<C, inv::EPI_ROWBIAS, inv::OUT_F32, inv::GRID_TILES, true>(p, dim3(ntiles), block, s);
            return hipGetLastError();
        }
        return hipErrorInvalidConfiguration;
    }
    if (mode == inv::GRID_SPLITK)
        ok = launch_epi<C, inv::GRID_SPLITK>(p, epi, out, dim3(ntiles * p.ksplit), block, s);
    else if (mode == inv::GRID_STREAMK)
        ok = launch_epi<C, inv::GRID_STREAMK>(p, epi, out, dim3((unsigned)p.ksplit), block, s);
    else
        ok = launch_epi<C, inv::GRID_TILES>(p, epi, out, dim3(ntiles), block, s);
    return ok ? hipGetLastError() : hipErrorInvalidConfiguration;
}

}  // namespace

#define INV_DEFINE_LAUNCH(id)                                                                               \
    hipError_t inv_gemm_launch_##id(const inv::GemmParams &p, int epi, int out, int mode, hipStream_t s) {   \
        return launch_cfg<INV_CFG_##id>(p, epi, out, mode, s);                                               \
    }
#define INV_EXPAND_DEFINE(id) INV_DEFINE_LAUNCH(id)
INV_EXPAND_DEFINE(INV_CFG_ID)
