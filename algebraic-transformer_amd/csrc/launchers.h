// Host launchers of the gfx950 kernels (defined in the *.hip translation units).
#pragma once

#include "attn_common.h"
#include "attn_prep.h"
#include "head_params.h"

namespace alg {

int attn_fwd_f32_query_block(int B, int H, int T);
hipError_t launch_attn_fwd(const AttnFwdParams& p, int D, bool bf16_io, int mode, hipStream_t st);
hipError_t launch_attn_bwd(const AttnBwdParams& p, int D, bool bf16_io, const int* modes, int nmodes,
                           hipStream_t st);
int attn_bwd_sink_blocks(int T);
int attn_prep_blocks(size_t rows);
hipError_t launch_attn_prep(const PrepParams& p, bool bf16_io, GuardParams g, hipStream_t st);
hipError_t launch_attn_guard(const GuardParams& g, hipStream_t st);
int attn_qk_prologue_blocks(int B, int H, int T, int D, bool bf16_io);
hipError_t launch_cayley_tables(const float* w, int half, int T, float* cos_out, float* sin_out, hipStream_t st);
hipError_t launch_attn_qk_prologue(const QkPrologueParams& p, bool bf16_io, GuardParams g, hipStream_t st);
hipError_t launch_attn_qk_prologue_bwd(const QkPrologueBwdParams& p, bool bf16_io, float* dq_gain, float* dk_gain,
                                       hipStream_t st);

int head_vocab_tiles(int V);
int head_token_pad(int N);
int head_vocab_pitch(int V);
int head_stat_blocks(int N);
int head_dh_split(int N, int d, int V);
int head_dh_kchunk(int V, int split);
struct HeadDePlan {
  int tiles, full, split, kchunk;
};
HeadDePlan head_de_plan(int N, int d, int V);
hipError_t launch_head_fwd(const HeadParams& p, hipStream_t st);
hipError_t launch_head_bwd(const HeadParams& p, hipStream_t st);
// Rows [v0, v0 + vc) of the vocabulary as a head of its own: E, E32 and dE offset, V = vc,
// targets compared with v + v0.
HeadParams head_vocab_chunk(const HeadParams& p, int v0, int vc);
hipError_t launch_head_bwd_streamed(const HeadParams& p, int chunk, hipStream_t st);
hipError_t launch_head_eval(const HeadParams& p, hipStream_t st);
hipError_t launch_head_stats(const HeadParams& p, int vocab_tiles, hipStream_t st);
hipError_t launch_head_eval_stats(const HeadParams& p, int vocab_tiles, hipStream_t st);
int head_f32_vocab_tiles(int V);
int head_f32_dh_split(int N, int d, int V);
int head_f32_dh_kchunk(int V, int split);
hipError_t launch_head_fwd_f32(const HeadParams& p, hipStream_t st);
hipError_t launch_head_bwd_f32(const HeadParams& p, hipStream_t st);
hipError_t launch_head_bwd_f32_streamed(const HeadParams& p, int chunk, hipStream_t st);
hipError_t launch_head_eval_f32(const HeadParams& p, hipStream_t st);
int rms_norm_max_d();
int rms_norm_blocks(int rows);
int rms_norm_gain_groups(int rows);
hipError_t launch_rms_norm_fwd(const RmsNormParams& p, hipStream_t st);
hipError_t launch_ffn_fwd(const FfnParams& p, hipStream_t st);
hipError_t launch_ffn_dy(const FfnParams& p, hipStream_t st);
struct FfnGemmPlan {
  int tiles, full, split, kchunk;
};
FfnGemmPlan ffn_gemm_plan(int M, int N, int K);
size_t ffn_gemm_workspace_bytes(const FfnGemmPlan& pl);
hipError_t launch_ffn_gemm(const FfnGemmParams& g, int a_mode, int b_mode, hipStream_t st);
hipError_t launch_rms_norm_bwd(const RmsNormParams& p, float* dgain, hipStream_t st);

}  // namespace alg
