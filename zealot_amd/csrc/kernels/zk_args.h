// zk_args.h — kernel argument blocks shared by the gfx950 code object and the
// host runtime. Plain structs (pointers, 32/64-bit scalars): the layout is
// identical on x86-64 and amdgcn, so the host passes them by value through
// hipModuleLaunchKernel.
#pragma once
#include <stdint.h>

namespace zk {

// zk_epoch_end: one block of 16 wavefronts (32 lane groups, one quantity
// each at a time).
constexpr int kFinalizeThreads = 1024;
// Block sizes of zk_actor_loss (32 lane groups) and zk_reduce_all (whose
// extra last block runs the minibatch tail with kReduceAllThreads / 32 lane
// groups).
constexpr int kLossThreads = 1024;
constexpr int kReduceAllThreads = 256;
static_assert(kReduceAllThreads % 64 == 0, "whole wavefronts");

enum EpiMode : int {
  kEpiStore = 0,    // C = acc
  kEpiBiasN = 1,    // C = act(acc + bias[n])           (batch-major forward)
  kEpiBiasM = 2,    // C = act(acc + bias[m*stride])    (feature-major forward)
  kEpiEluGrad = 3,  // C = acc * elu'(Y[m*ldy + n])     (dgrad of a hidden layer)
};

struct GemmArgs {
  const float* A;
  const float* B;
  float* C;
  const float* bias;
  const float* Y;
  float* rowsumA;          // [splits x M] row sums of A (n-tile-0 blocks), nullable
  const int* permA;        // storage-row gather for A, nullable
  const int* permB;        // storage-row gather for B, nullable
  const int* guard;        // no-op when *guard == 0, nullable
  long long split_stride;  // elements between split-K partial outputs
  int M, N, K;
  int lda, ldb, ldc, ldy;
  int bias_stride;
  int epi;
  int act;                 // ELU in the bias epilogues
  int vecA, vecB;          // float4 global loads are aligned and in bounds
  int kt_per_split;        // k-tiles per split-K slice (narrow weight gradient: rows)
  int nsplit;              // split-K slices of this problem
};

// Up to two GEMMs of one kernel variant in one launch (the actor's and the
// critic's layer). Tiled kernels: a 1-D grid in which problem i owns blocks
// [blk0[i], blk0[i] + gx[i] * gy[i] * gz[i]), laid out as its own tile grid
// gx x gy with gz split-K slices, so problems of different shapes share a
// launch without idle blocks. Narrow kernels: grid.z = problem (zper = 1),
// blocks outside a problem's grid return at once.
constexpr int kMaxGemmBatch = 2;
struct GemmBatch {
  GemmArgs g[kMaxGemmBatch];
  int count;
  int zper;
  int blk0[kMaxGemmBatch];
  int gx[kMaxGemmBatch], gy[kMaxGemmBatch], gz[kMaxGemmBatch];
};

// A layer's weight-gradient batch and data-gradient batch as one launch: the
// weight-gradient batch's nw blocks first, then the data-gradient batch's.
struct GemmPair {
  GemmBatch w, d;
  int nw;
};

struct SplitReduceArgs {
  const float* part;     // [splits x rows_mn x cols] dense partials
  float* out;            // element (r, c) at out[r * ldo + c]
  const float* rowpart;  // [splits x rows], nullable
  float* rowout;         // [rows]
  const int* guard;
  long long mn;          // rows_mn * cols
  int cols, ldo;
  int rows;
  int splits;
  int lanes;  // split lanes per output element: a power of two in [1, 256]
};

// One output tensor of the all-layer reduction (zk_reduce_all): the fixed-
// order sum over `splits` dense partial slices (part, rowpart), or, with
// part == nullptr, a tensor already final in `out` / `rowout` that only
// contributes its sum of squares. Blocks [blk0, blk0 + nqb) cover the matrix
// in float4 quads, the next nrb blocks the row sums; `lanes` split lanes per
// output element (a power of two, 256 / lanes outputs per block).
struct ReduceSeg {
  const float* part;
  const float* rowpart;
  float* out;
  float* rowout;
  long long mn;
  int cols, ldo, rows, splits, lanes;
  int blk0, nqb, nrb;
};

// Scalars that live on the device for a whole update so that no kernel needs
// a host round trip (learning rate, Adam step, clip scales, statistics).
struct DevState {
  float lr;
  int t;                     // Adam steps taken (ActorCritic::update semantics)
  float bc1, bc2;            // bias corrections for the next Adam launch
  float scale[3];            // clip scale per group: actor, critic, log_std
  int active;                // 0 once the trainer's KL early stop fired
  int epochs_run;
  int mb_in_epoch;
  float ep_kl, ep_surr, ep_vloss, ep_ent;
  float stats[5];            // kl, surrogate, value_loss, entropy, lr
  float last_kl;
  float norm[3];             // last pre-clip norms (actor, critic, log_std) / global
  int pad0;
  unsigned long long gstep;  // trainer gstep (src/bin/biped_train_gpu.rs:1165)
};

struct PpoParams {
  int mode;  // 0 = ActorCritic::update (zealot-rl/src/ppo.rs:338), 1 = GPU trainer
  int A;     // action dim
  int mb;    // rows per minibatch
  int n_mb;  // minibatches per epoch
  float clip, entropy_coef, value_coef, scale;  // scale = 1/mb
  float max_grad_norm;
  float desired_kl, lr_min, lr_max;
  int adaptive_lr, early_stop;
  int clamp_ls;  // clamp log_std to [-1.6, 1.0] in every Adam step
  float beta1, beta2, eps;
};

// The scalar tail of a minibatch step that needs only the loss partials
// (statistics, the log_std gradient and its squared norm, the Adam step
// count and the lr rule): run by one extra block of zk_reduce_all, beside the
// gradient reduction; the clip scales, which need every block's squared-norm
// partial, are taken by zk_adam's blocks (AdamArgs::clip).
struct FinalizeArgs {
  DevState* st;
  const float* gls_part;    // [A x nb_a]
  const float* astat_part;  // [2 x nb_a]
  const float* vstat_part;  // [nb_v]
  float* sq_part;           // slot nsq receives the log_std gradient's squared norm
  const float* log_std;     // [A] (pre-step values)
  float* g_logstd;          // [A] log_std gradient slot in the flat gradient
  PpoParams pp;
  int nb_a, nb_v, nsq;
};

constexpr int kMaxReduceSegs = 16;
struct ReduceAllArgs {
  ReduceSeg seg[kMaxReduceSegs];
  int nseg;
  float* sq_part;  // per-block sum of squares of the block's final values
  const int* guard;
  int tail_block;  // >= 0: this block (the last) runs the minibatch tail `tail`
  FinalizeArgs tail;
};

struct ActorLossArgs {
  const float* mean;      // [rows x ldm] actor output of this minibatch
  const float* action;    // [n x ldact] full batch
  const float* adv;       // [n]
  const float* logp_old;  // [n]
  const float* mean_old;  // [n x ldmo], nullable (no KL statistic)
  const float* log_std;   // [A]
  const int* perm;        // sample = perm ? perm[row0 + r] : row0 + r
  float* delta;           // [rows x ldd] dL/dmean
  float* gls_part;        // [A x blocks] log_std gradient partials (component-major)
  float* stat_part;       // [2 x blocks] surrogate, kl partials
  const int* guard;
  // Element (row r, component k) of mean / action / mean_old / delta is at
  // r * ld + k * c: batch-major (c = 1) or feature-major (ld = 1, c = the
  // feature stride).
  int ldm, ldact, ldmo, ldd;
  int cm, cact, cmo, cdd;
  int row0, rows, A;
  int rows_per_block;  // samples handled by one block
  int group;           // lanes per sample: 32 (A <= 32) or 64 (A <= 64)
  float clip, entropy_coef, scale;
};

struct ValueLossArgs {
  const float* v;          // [rows x ldv] critic output
  const float* value_old;  // [n]
  const float* ret;        // [n]
  const int* perm;
  float* delta;            // [rows x ldd]
  float* stat_part;        // [blocks] value-loss partials
  const int* guard;
  int ldv, ldd, row0, rows;
  float clip, value_coef, scale;
};

// zk_head: the output layer of both nets fused with the PPO losses for one
// minibatch (blockIdx.z: 0 actor, 1 critic). Tiles of kHeadRows rows are
// strided over the blocks of a net; the last hidden width is at most
// kHeadMaxHidden and the action dim at most kHeadMaxActions.
constexpr int kHeadRows = 64;
constexpr int kHeadThreads = 512;  // 8 wavefronts per block
constexpr int kHeadMaxBlocks = 512;
constexpr int kHeadMaxHidden = 128;
constexpr int kHeadMaxActions = 32;
struct HeadNet {
  const float* x;  // [rows x ldx] last hidden activations (after ELU)
  const float* w;  // [nout x ldw] output-layer weights
  const float* b;  // [nout]
  float* out;      // [rows x ldo] output (actor mean / critic value)
  float* dz;       // [rows x ldz] dL/dz of the last hidden layer
  float* wpart;    // [blocks x nout x H] weight-gradient partials
  float* bpart;    // [blocks x nout] bias-gradient partials
  int ldx, ldw, ldo, ldz, H;
  // zk_head_fwd*: the tile of x is computed in the block instead of read,
  // x = ELU(x2 . w2^T + b2) — the last hidden layer's forward (x2 [rows x
  // ldx2] its input, w2 [H x ldw2] its weights, k2 its input width).
  const float* x2;
  const float* w2;
  const float* b2;
  int ldx2, ldw2, k2;
};
struct HeadArgs {
  HeadNet net[2];
  const float* action;    // [n x ldact]
  const float* logp_old;  // [n]
  const float* adv;       // [n]
  const float* mean_old;  // [n x ldmo], nullable
  const float* log_std;   // [A]
  const float* value_old; // [n]
  const float* ret;       // [n]
  const int* perm;        // sample = perm ? perm[row0 + r] : row0 + r
  float* gls_part;        // [A x blocks] log_std gradient partials
  float* astat_part;      // [2 x blocks] surrogate, kl partials
  float* vstat_part;      // [critic_blocks] value-loss partials
  float* kl_part;         // [A x blocks] sums of (mean - mean_old)^2 per component, nullable
  const int* guard;
  long long rows;
  // Actor: block x (of gridDim.x) takes tiles x, x + gridDim.x, ... (at most
  // tiles_per_block). Critic: blocks x < critic_blocks take tiles x,
  // x + critic_blocks, ... (at most critic_tiles), the others exit at once.
  int row0, A, ldact, ldmo, tiles_per_block;
  int critic_blocks, critic_tiles;
  float clip, entropy_coef, value_coef, scale;
};

struct SumsqArgs {
  const float* x;
  float* part;           // one partial per block
  const int* guard;
  long long off0, len0;  // group 0 range
  long long off1, len1;  // group 1 range
  int blocks0;           // blocks assigned to group 0; the rest cover group 1
  int chunk;             // elements per block
};

struct AdamArgs {
  float* p;
  const float* g;
  float* m;
  float* v;
  DevState* st;               // lr / bc1 / bc2 (and with clip 0 the scales) from the device, or
  const int* guard;
  long long n, end_a, end_c;  // groups: [0,end_a) actor, [end_a,end_c) critic, rest log_std
  float lr, bc1, bc2;         // ... these when st == nullptr (scale = 1)
  float beta1, beta2, eps;
  int clamp_ls;               // clamp group 2 to [-1.6, 1.0] (ppo.rs:508)
  // Clip scales taken here from zk_reduce_all's squared-norm partials (every
  // block sums them in the same fixed order; block 0 records scales and
  // norms in st): clip 0 = st->scale as it is; 1 = per net (ActorCritic:
  // partials [0, nsq_a) actor, [nsq_a, nsq) critic, log_std unclipped);
  // 2 = one global scale over actor + critic + log_std (sq_part[nsq]).
  const float* sq_part;
  int nsq_a, nsq, clip;
  float max_grad_norm;
};

struct EpochBeginArgs {
  DevState* st;
  const int* guard;
  PpoParams pp;
};

struct KlArgs {
  const float* mean;         // [rows x ldm] last minibatch's actor output
  const float* mean_old;     // [n x ldmo]
  const float* log_std;      // [A] current
  const float* log_std_old;  // [A] rollout snapshot
  const int* perm;
  float* part;               // [blocks]
  const int* guard;
  int ldm, ldmo, row0, rows, A;
};

// kl_form 0: kl_part holds the per-block KL totals of zk_kl. kl_form 1: it
// holds zk_head's [A x nkl] per-component sums of (mean - mean_old)^2 over
// the last minibatch, combined with log_std / log_std_old here.
struct EpochEndArgs {
  DevState* st;
  const float* kl_part;      // trainer mode, nullable
  const float* log_std;      // [A] current (kl_form 1)
  const float* log_std_old;  // [A] rollout snapshot (kl_form 1)
  int* active;               // early-stop flag (the guard of every later kernel)
  PpoParams pp;
  int nkl;
  int kl_form;
  int begin_next;            // also open the next epoch (zk_epoch_begin) if still active
};

// zk_gae: one wavefront per block (envs spread over the CUs); trajectories
// of up to kGaeMaxT steps are scanned from registers.
constexpr int kGaeThreads = 64;
constexpr int kGaeMaxT = 32;
struct GaeArgs {
  const float* r;
  const float* v;
  const uint8_t* done;
  const float* last_v;       // [N]
  float* adv;
  float* ret;
  long long in_ts, in_es;    // element (t, e) of r / v / done at t*in_ts + e*in_es
  long long out_ts, out_es;  // element (t, e) of adv / ret
  int T, N;
  float gamma, lam;
  const int* guard;
};

struct AdvNormArgs {
  float* x;
  float* part;   // [nparts] sums
  float* part2;  // [nparts] sums of squared deviations
  const int* guard;
  long long n;
  int nparts;
  int chunk;     // elements per block
  int phase;     // 0: sums, 1: squared deviations, 2: apply
  float* const* wb;  // nullable: phase 2 also writes the result to *wb (device-resident pointer)
};

struct EluBwdArgs {
  float* g;
  const float* y;
  long long rows;
  int cols, ldg, ldy;
  const int* guard;
};

struct RowSumArgs {
  float* out;
  const float* x;
  int rows, cols, ldx;
  const int* guard;
};

struct CopyRowsArgs {
  float* dst;
  const float* src;
  const int* perm;  // source row = perm ? perm[row0 + r] : row0 + r
  long long rows;
  int cols, ldd, lds, row0;
  int zero_pad;     // write 0 to columns [cols, ldd); otherwise leave them
  const int* guard;
};

// zk_transpose: dst[j * ldd + i] = src[i * lds + j] for i < rows, j < cols,
// 64 x 64 tiles through LDS (grid x over column tiles, y over row tiles).
constexpr int kTransposeTile = 64;
struct TransposeArgs {
  const float* src;
  float* dst;
  long long rows, cols, lds, ldd;
};

struct SampleArgs {
  const float* mean;  // [rows x ldm]
  const float* log_std;
  const float* eps;   // [rows x lde]
  float* action;      // [rows x lda]
  float* logp;        // [rows]
  int rows, A, ldm, lde, lda;
  const int* guard;
};

// One rollout step in one launch (zk_policy): per block kPolicyRows rows, grid
// (row blocks, nets). Net 0 is the actor, net 1 (when present) the critic.
// Each block normalises its rows of x with the net's Normalizer state (when
// norm is set), runs every layer with the activations in LDS and writes the
// last layer to out (when set); with `sample`, the actor's blocks then draw
// action = mean + exp(log_std) * eps and its log-probability. Hidden widths
// are multiples of 16 up to kPolicyMaxWidth, the input padded to a multiple
// of 16 within the layer-0 weight rows, and the output width at most 32
// (the host checks).
constexpr int kPolicyRows = 16;
constexpr int kPolicyThreads = 1024;  // 16 wavefronts: at most two 16-column tiles each
constexpr int kPolicyMaxWidth = 512;
constexpr int kPolicyMaxLayers = 8;
struct PolicyNet {
  const float* x;     // [rows x ldx] inputs (raw, or already normalised)
  const float* norm;  // Normalizer state [2 * dims[0] + 1], nullable
  float* out;         // [rows x ldo] the last layer's output, nullable
  const float* wp;    // the net's weights in the zk_policy_pack layout; layer l at wp + wp_off[l]
  long long wp_off[kPolicyMaxLayers], b_off[kPolicyMaxLayers];
  int dims[kPolicyMaxLayers + 1];
  int L, ldx, ldo;
};
// zk_policy_pack: the weights zk_policy reads, rewritten from the flat
// parameter rows ([N x ldw] per layer) so that one wavefront's load of a
// 16-column tile's 16-wide reduction chunk is 1 KB of consecutive floats:
// per tile T and chunk c, 256 floats in which lane L's float4 is
// W[16 T + L % 16][16 c + 4 (L / 16) .. + 3], zero past N rows and K columns
// (K the layer's input width; kc = ceil(K / 16) chunks). One segment per
// (net, layer); segment s covers float4 indices [q0, next q0) of the output.
constexpr int kPolicyPackSegs = 2 * kPolicyMaxLayers;
struct PolicyPackSeg {
  long long src;  // the layer's weight rows in params
  long long dst;  // its packed block in dst
  long long q0;   // first float4 index of the segment
  int ldw, N, K, kc;
};
struct PolicyPackArgs {
  const float* params;
  float* dst;
  PolicyPackSeg seg[kPolicyPackSegs];
  int nseg;
  long long nq;  // float4 outputs over all segments
};
struct PolicyArgs {
  PolicyNet net[2];
  const float* params;
  const float* log_std;  // [A]
  const float* eps;      // [rows x lde]
  float* action;         // [rows x lda]
  float* logp;           // [rows]
  long long rows;
  int A, lde, lda, sample;
};

// Observation normaliser (Normalizer / PendingNorm, zealot-rl/src/ppo.rs:104-206).
// A state is float[2 * dim + 1]: mean[dim], m2[dim], count; a pending state
// with count 0 is empty (its mean and m2 are zero).
constexpr int kNormMaxDim = 4096;
constexpr int kNormChunkRows = 256;    // rows per partial-statistics chunk
constexpr int kNormFoldThreads = 1024;  // zk_norm_merge / zk_norm_commit block
struct NormArgs {
  const float* x;   // [rows x ldx]
  float* out;       // zk_norm_apply: [rows x ldo]
  float* state;     // fold / commit target, zk_norm_apply source, zk_norm_set target
  float* pending;   // zk_norm_commit: folded into state, then emptied
  float* part;      // [nchunks x 2 x dim]: per chunk mean[dim], then M2[dim]
  long long rows;
  int dim, ldx, ldo, nchunks;
  int rows_per_block;  // zk_norm_apply
  int unit_prior;   // zk_norm_set: 1 = Normalizer::new, 0 = empty pending state
};

struct ClampArgs {
  float* x;
  int n;
  float lo, hi;
  const int* guard;
};

// The caller's pointers of one rollout batch, uploaded to device memory with
// every update so that a captured update graph reads them at replay time
// instead of baking them in (zk_stage, and the advantage write-back).
struct BatchPtrs {
  const float* mat[4];  // obs, critic_obs, action, mean_old (nullable)
  const float* vec[4];  // logp_old, value_old, adv, ret
  float* adv_out;       // the caller's adv: normalised advantages are written back
};

// zk_stage: copies batch fields into library-owned batch-major buffers.
// A matrix job moves tiles of kStageRows samples x kStageCols features; a
// feature-major source (element (sample i, feature k) at k * ld + i) is
// transposed through LDS, a batch-major one (i * ld + k) copied row by row;
// columns [cols, ldd) of the destination are written as zeros. A vector job
// moves kStageVec elements per block. Blocks [blk0, blk0 + blocks) of the
// 1-D grid belong to a job.
constexpr int kStageRows = 64;
constexpr int kStageCols = 32;
constexpr int kStageVec = 2048;
constexpr int kMaxStageJobs = 8;
struct StageJob {
  float* dst;    // [rows x ldd]
  long long ld;  // source stride (row stride, or feature stride when fm)
  int cols, ldd;
  int fm;        // source is feature-major
  int slot;      // BatchPtrs::mat[slot] (matrix job) or vec[slot] (vector job)
  int vec;
  int tiles_c;   // column tiles of a matrix job
  int blk0, blocks;
};
struct StageArgs {
  const BatchPtrs* ptrs;
  const int* perm;  // source row of staged row r = perm ? perm[row0 + r] : row0 + r
  const int* guard;
  long long rows, row0;
  StageJob job[kMaxStageJobs];
  int njobs;
};

// Sum of squares over a list of tensors (zk_sumsq_multi): blocks [blk0[j],
// blk0[j + 1]) cover tensor j in chunks of `chunk` elements, one partial per
// block; zk_clip_scale then adds the partials in block order, takes the norm
// and the clip scale.
constexpr int kMaxNormTensors = 48;
struct SumsqMultiArgs {
  const float* x[kMaxNormTensors];
  long long n[kMaxNormTensors];
  int blk0[kMaxNormTensors + 1];
  int count, chunk;
  float* part;  // one partial per block
};
struct ClipScaleArgs {
  const float* part;
  int nparts;
  float max_norm;  // <= 0: scale 1
  float* scale;    // [1] max_norm / norm when norm > max_norm, else 1
  float* norm;     // [1] nullable
};

// Adam over a list of tensors in one launch (zk_adam_multi): blocks
// [blk0[j], blk0[j + 1]) cover tensor j, 4 elements per thread; the gradient
// is multiplied by *scale first when scale is set.
constexpr int kMaxAdamTensors = 48;
struct AdamTensor {
  float* p;
  const float* g;
  float* m;
  float* v;
  long long n;
};
struct AdamMultiArgs {
  AdamTensor t[kMaxAdamTensors];
  int blk0[kMaxAdamTensors + 1];
  int count;
  const float* scale;  // nullable
  float lr, bc1, bc2, beta1, beta2, eps;
  // With `part` set, every block takes the clip scale itself from the
  // zk_sumsq_multi partials (nparts, added in zk_clip_scale's order, the
  // same rule) instead of reading `scale`; block 0 writes it and the norm
  // to scale_out / norm_out (nullable).
  const float* part;
  int nparts;
  float max_norm;
  float* scale_out;
  float* norm_out;
};

}  // namespace zk
