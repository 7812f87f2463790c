// Host-callable launchers of the HIP kernels (one .hip file each).
#pragma once

#include <hip/hip_runtime_api.h>

#include "common.h"
#include "vm.h"

namespace rew {

// ---- fused elementwise (k_ew.hip) ------------------------------------------
// `vec`: the innermost space dim is a multiple of vm::kVec and every
// LM_CONTIG leaf / output is vector-aligned.
void launch_ew(const vm::Program& P, const vm::Space& S, bool vec,
               hipStream_t stream);

// ---- run-time compiled programs (jit.cpp) ------------------------------------
// Launch P as a hipRTC-compiled kernel specialised to its constants; false
// when compiled kernels are off or the program failed to compile (the
// caller then runs the interpreter).
struct ReduceArgs;
bool jit_launch_ew(const vm::Program& P, const vm::Space& S, bool vec, hipStream_t stream);
bool jit_launch_reduce(const vm::Program& P, const vm::Space& S, const ReduceArgs& A, bool vec,
                       hipStream_t stream);
// Launches so far (process-wide) that reused an already compiled program;
// programs compiled by hipRTC and programs loaded from the persistent cache.
int64_t jit_cache_hits();
int64_t jit_programs_compiled();
int64_t jit_programs_loaded();

// ---- reductions (k_reduce.hip) ---------------------------------------------
enum RedOp : int {
  RED_SUM = 0, RED_MAX, RED_MIN, RED_PROD, RED_AND, RED_OR, RED_MAXI, RED_MINI
};
struct ReduceArgs {
  int op;
  uint32_t n_out;   // product of kept dims
  uint32_t n_red;   // product of reduced dims
  void* out;
  int out_dtype;
  // further reductions of the same values in the same pass (rew's
  // reduceSum and reduceMax of one tensor over the same axes), each into its
  // own output of out_dtype; every op accumulates in the single-op order
  int n_extra = 0;
  int extra_op[3] = {0, 0, 0};
  void* extra_out[3] = {nullptr, nullptr, nullptr};
  // reduceMean's divide (src/rew/ops/reduce.nim:132-150) at the store: f32
  // output mean_out[i] = acc / mean_div[i] (IEEE fp32 division) of
  // accumulator mean_src[i] (0: the main op, x: extra op x - 1), a RED_SUM
  // with out_dtype f32
  int n_mean = 0;
  int mean_src[2] = {0, 0};
  float mean_div[2] = {1.0f, 1.0f};
  void* mean_out[2] = {nullptr, nullptr};
};
// Space = [kept..., reduced...]; program output 0 names the value register.
void launch_reduce(const vm::Program& P, const vm::Space& S,
                   const ReduceArgs& A, bool vec, hipStream_t stream);

// ---- dot_general as a batched GEMM (k_gemm.hip) ------------------------------
// C[b, m, n] = sum_k A[b, m, k] * B[b, k, n]; all strides in elements.
// Dense C with row pitch ldc = N unless c_sm says otherwise.
struct GemmArgs {
  const void* a;
  const void* b;
  void* c;
  int dtype;       // operand dtype (bf16 / f16 / f32)
  int c_dtype;     // result dtype
  int64_t batch, M, N, K;
  int64_t a_sb, a_sm, a_sk;
  int64_t b_sb, b_sk, b_sn;
  int64_t c_sb, c_sm;
  // Fused epilogue (rew's Linear.forward bias add, the decoder's residual
  // add, GatedFeedForward's SiLU gate), each rounded like the op sequence:
  //   EPI_BIAS      c = rnd(rnd(acc) + bias[n])
  //   EPI_BIAS_RES  c = rnd(res[b,m,n] + rnd(rnd(acc) + bias[n]))
  //   EPI_SWIGLU    dual GEMM with B and b2: g = rnd(rnd(acc) + bias[n]),
  //                 u = rnd(rnd(acc2) + bias2[n]),
  //                 c = bf16(g * (1 / (1 + exp(-g))) * u)   (fp32 ops)
  // rnd() rounds to c_dtype; bias / res / c share c_dtype.
  int epi;
  const void* bias;
  const void* bias2;
  const void* res;
  int64_t res_sb, res_sm;
  const void* b2;
  // EPI_BIAS_ROPE (bf16, batch 1): y = rnd(rnd(acc) + bias[n]) as EPI_BIAS,
  // then rew's applyRotate on the adjacent pairs (2i, 2i+1) of each head
  // (src/rew/nn/rope.nim:56-108): with row m = b * rope_S + s and column
  // n = h * rope_D + d,
  //   c = rope_cos[t], sn = rope_sin[t], t = b tb + s ts + h th + (d / 2) ti
  //   out[d] = bf16(c y[d] - sn y[d+1]),  out[d+1] = bf16(sn y[d] + c y[d+1])
  // (each product and sum rounded to fp32), stored at
  //   c + b out_b + s out_s + h out_h + d   (c_sm / c_sb unused).
  const float* rope_cos;
  const float* rope_sin;
  int64_t rope_S, rope_D;
  int64_t rope_tb, rope_ts, rope_th, rope_ti;
  int64_t out_b, out_s, out_h;
  // EPI_BIAS_RELU (the f32 kernels that store through epi_value): rew's relu
  // after the bias add, c = maximum(y, relu_c) (relu_first) or
  // maximum(relu_c, y), NaN-propagating with the VM's zero-sign rule
  float relu_c;
  int relu_first;
};
enum GemmEpi : int {
  EPI_NONE = 0, EPI_BIAS = 1, EPI_BIAS_RES = 2, EPI_SWIGLU = 3, EPI_BIAS_ROPE = 4,
  EPI_BIAS_RELU = 5
};
void launch_gemm(const GemmArgs& g, hipStream_t stream);

// Grouped GEMM over packed rows (the routed experts of a MoE layer).  Group
// i owns packed rows [off[i], off[i+1]) and row tiles
// [mt_start[i], mt_start[i+1]); its B / b2 / bias / bias2 come from the
// device pointer tables.  Row r of the A operand is A row rows[r] when
// `rows` is set (a gather from the token matrix), else packed row r.  C is
// written at its packed row.  The per-element arithmetic is the 256x256
// kernel's (same MFMA sequence over the same k order), so a group's rows
// equal the dense GEMM's rows bit for bit.  Fields of GemmArgs keep their
// meaning except: a = the A matrix (token matrix when gathering) with M its
// row count; b, b2, bias, bias2 ignored (taken from the tables); c = the
// packed output with c_sm its row stride.
//
// A group of at most kSmallGroupRows rows is cut into kSmallTileM-row tiles
// (the LDS kernel runs those with its four waves side by side on 64 rows, a
// quarter of the MFMAs of a 256-row tile), any other group into 256-row
// tiles: group_tiles gives the count the routing writes into mt_start, and
// every grouped kernel reads a group's tile height back by group_tile_rows.
constexpr int kSmallGroupRows = 128;
constexpr int kSmallTileM = 64;
constexpr int group_tile_rows(int64_t rows) { return rows <= kSmallGroupRows ? kSmallTileM : 256; }
constexpr int group_tiles(int64_t rows) {
  return (int)((rows + group_tile_rows(rows) - 1) / group_tile_rows(rows));
}
struct GroupArgs {
  const int32_t* off;       // n_groups + 1 (device)
  const int32_t* mt_start;  // n_groups + 1 (device)
  const int32_t* rows;      // packed row -> A row, or nullptr
  int n_groups;
  int64_t max_mtiles;       // grid bound on mt_start[n_groups]
  const void* const* b;     // n_groups device pointers each
  const void* const* b2;
  const void* const* bias;
  const void* const* bias2;
  // host side: the largest |b2[i] - b[i]| in bytes (the dual B operands
  // share one buffer descriptor when it is small), -1 when not known
  int64_t dual_span = -1;
};
// Whether launch_gemm_grouped can run g (dtype, layout, epilogue, 32-bit
// buffer extents).
bool gemm_grouped_ok(const GemmArgs& g);
void launch_gemm_grouped(const GemmArgs& g, const GroupArgs& ga, hipStream_t stream);

// The direct-to-LDS 256x256 kernels (k_gemm_lds.hip): bf16 in / out, any
// epilogue; *b_kc reports whether B is K-contiguous.  `ga` non-null runs
// the grouped mode.
bool gemm_lds_ok(const GemmArgs& g, bool* b_kc);
void launch_gemm_lds(const GemmArgs& g, const GroupArgs* ga, hipStream_t stream);
// Up to kMaxSegs GEMMs over one A matrix (same a, M, K, strides) in one
// launch: segment i owns the output-column tiles [tn0[i], tn0[i + 1]) and
// keeps its own B, bias, C and epilogue (EPI_NONE / EPI_BIAS /
// EPI_BIAS_RES / EPI_BIAS_ROPE).  gemm_multi_ok checks that the set can run.
constexpr int kMaxSegs = 3;
struct GemmSegs {
  int n;
  int64_t tn0[kMaxSegs + 1];
  GemmArgs g[kMaxSegs];
};
bool gemm_multi_ok(const GemmArgs* segs, int n);
void launch_gemm_multi(const GemmArgs* segs, int n, hipStream_t stream);
// Whether launch_gemm runs g with its epilogue (EPI_SWIGLU needs the large
// dual kernel; the others run on every MFMA kernel).
bool gemm_epilogue_ok(const GemmArgs& g);
// Name of the kernel variant launch_gemm would pick (for profiles/tests).
const char* gemm_variant(const GemmArgs& g);

// ---- gather (k_gather.hip) ---------------------------------------------------
// torch_index_select with batch_dims = 0: out[pre, i, post] =
// operand[pre, index[i], post]; rows of `row_bytes` contiguous bytes.
struct GatherArgs {
  const void* src;
  const void* index;
  void* out;
  int index_dtype;
  int64_t n_pre;        // product of operand dims before `dim`
  int64_t src_dim;      // operand.shape[dim]
  int64_t n_idx;        // number of indices
  int64_t row_bytes;    // product of operand dims after `dim` * elem size
};
void launch_gather(const GatherArgs& g, hipStream_t stream);

// stablehlo.gather / stablehlo.scatter over dense row-major tensors of rank
// <= 8 (src/rew/ops/gather.nim:10-28, scatter.nim:10-39; the StableHLO
// dimension-number semantics).  One thread per element of the iteration
// space (gather: the result; scatter: the updates).  The host resolves the
// dimension numbers into roles:
//   role[d] >= 0   iteration dim d is a window dim: it offsets x dim role[d]
//   role[d] = -1-k iteration dim d is batch dim k of the index tensor
// The index vector of an element is index[sum_k c_k * stride_idx_batch[k] +
// j * stride_idx_vec], j < n_map, and sets the start of x dim map_x[j];
// x dim bat_x[i] starts at the iteration coordinate of dim bat_it[i]
// (operand / input batching dims).  Gather clamps every start into
// [0, dims_x - slice]; scatter skips an update whose index falls outside x.
constexpr int kScatterReplace = 0, kScatterAdd = 1, kScatterMax = 2, kScatterMin = 3,
              kScatterMul = 4;
struct IndexMapArgs {
  const void* src;    // gather: operand; scatter: updates
  const void* index;
  void* out;          // gather: result; scatter: result, pre-filled with the input
  int esize, dtype, index_dtype;
  int op;             // scatter update computation (kScatter*)
  int clamp;          // 1: gather, 0: scatter
  int rank_it, rank_x;
  int64_t dims_it[8];
  int64_t dims_x[8], stride_x[8];
  int role[8];
  int64_t stride_idx_batch[8];
  int64_t stride_idx_vec;
  int n_map;
  int map_x[8];
  int n_bat;
  int bat_x[8], bat_it[8];
  int64_t slice[8];
  int64_t total;      // elements of the iteration space
};
void launch_gather_nd(const IndexMapArgs& g, hipStream_t stream);

// ---- pad / dynamicSlice / dynamicUpdateSlice (k_gather.hip) ---------------------
// One thread per result element over dense row-major tensors of rank <= 8.
//   pad:    out[o] = x[(o - lo) / step] where every dim's o - lo is a
//           non-negative multiple of step (= interior + 1) inside x, else
//           the padding value *y (negative lo / high crop);
//   slice:  out[o] = x[o + s], s the start scalars clamped to [0, x - out];
//   update: out[o] = y[o - s] inside the update window, else x[o], s clamped
//           to [0, x - y].
// Start scalars are read on the device (any integer dtype), so no value
// leaves the GPU.
enum { kWinPad = 0, kWinSlice = 1, kWinUpdate = 2 };
struct WindowArgs {
  int mode, esize, rank;
  const void* x;
  const void* y;  // pad: the padding value; update: the update tensor
  void* out;
  int64_t out_dims[8], x_dims[8], y_dims[8];
  int64_t lo[8], step[8];
  const void* start[8];
  int start_dt[8];
  int64_t total;
};
void launch_window(const WindowArgs& a, hipStream_t stream);

// ---- cholesky (k_gather.hip) --------------------------------------------------------
// Batched Cholesky factorisation of dense [batch, n, n] f32 / f64 matrices,
// one workgroup per matrix held in LDS (n <= kCholMaxN): A = L L^T from the
// lower triangle (lower) or A = U^T U from the upper one; the other
// triangle of the result is zero.  A matrix that is not positive definite
// gives NaN from the first failing pivot on.
constexpr int64_t kCholMaxN = 64;
struct CholeskyArgs {
  const void* x;
  void* out;
  int64_t batch, n;
  int f64, lower;
};
void launch_cholesky(const CholeskyArgs& a, hipStream_t stream);

// ---- triangular solve (k_gather.hip) -------------------------------------------------
// stablehlo.triangular_solve over [batch, n, n] a and b of [batch, n, m]
// (left_side: op(a) x = b) or [batch, m, n] (x op(a) = b), f32 / f64, n <=
// kCholMaxN: op(a) is a or its transpose (real adjoint = transpose), only the
// `lower` (or upper) triangle of a is read, and unit_diagonal takes its
// diagonal as ones.  One workgroup per matrix, a in LDS, one thread per
// right-hand side by substitution with the sums in k order.
struct TriSolveArgs {
  const void* a;
  const void* b;
  void* out;
  int64_t batch, n, m;
  int f64, left, lower, unit, trans;
};
void launch_trisolve(const TriSolveArgs& a, hipStream_t stream);

// ---- complex parts and the discrete Fourier transform (k_gather.hip) -----------------
// complex(re, im) interleaves two f32 / f64 tensors into c64 / c128; real / imag
// take a component (or, of a real tensor, the tensor / zeros).  mode: 0 complex,
// 1 real part, 2 imaginary part, 3 copy, 4 zeros; esize: component bytes.
struct ComplexArgs {
  const void* x;
  const void* y;
  void* out;
  int64_t n;  // result elements
  int esize, mode;
};
void launch_complex(const ComplexArgs& a, hipStream_t stream);
// One-axis DFT of [outer, len_in, inner] into [outer, len_out, inner], a thread
// per result element summing in double with twiddles exp(-+2 pi i k j / n) from
// (k j mod n): mode 0 complex forward, 1 complex inverse (scaled 1/n), 2 real to
// complex (len_out = n / 2 + 1), 3 complex to real (len_in = n / 2 + 1, the
// spectrum taken as Hermitian: the imaginary parts of bins 0 and n / 2 are not
// read).  f64: c128 / f64 data, else c64 / f32.
struct Fft1Args {
  const void* x;
  void* out;
  int64_t outer, inner, len_in, len_out, n;
  int f64, mode;
};
void launch_fft1(const Fft1Args& a, hipStream_t stream);

// ---- batch norm (k_gather.hip) -------------------------------------------------------
// stablehlo.batch_norm_{inference,training,grad} over x viewed as dense
// [outer, C, inner] (C at feature_index), f32 or f64, N = outer inner:
//   inference: y = scale (x - mean) / sqrt(var + eps) + offset   (out0)
//   training:  mean = sum x / N, var = sum (x - mean)^2 / N (out1, out2),
//              then y as inference                                (out0)
//   grad:      xn = (x - mean) / sqrt(var + eps); d_offset = sum dy (out2),
//              d_scale = sum dy xn (out1), dx = scale / sqrt(var + eps)
//              (dy - d_offset / N - xn d_scale / N)               (out0)
// Inference runs a thread per element, the others a workgroup per feature.
enum { kBnInference = 0, kBnTraining = 1, kBnGrad = 2 };
struct BatchNormArgs {
  int mode, f64;
  const void *x, *scale, *offset, *mean, *var, *dy;
  void *out0, *out1, *out2;
  int64_t outer, C, inner;
  double eps;
};
void launch_batchnorm(const BatchNormArgs& a, hipStream_t stream);
void launch_scatter(const IndexMapArgs& g, hipStream_t stream);

// ---- argmax / topK (k_select.hip) ----------------------------------------------
// argmax over dim n of x viewed as dense [outer, n, inner] f32; out [outer, inner]
// int32 (lowest index of the maximum; INT32_MAX where the slice holds NaN).
struct ArgmaxArgs {
  const float* x;
  int32_t* out;
  int64_t outer, n, inner;
};
void launch_argmax(const ArgmaxArgs& g, hipStream_t stream);

// ---- mixture-of-experts router (k_router.hip) -----------------------------------
// ids / vals = topK(softmax(x W + b), k) per token row (largest first, NaN
// last, lower column on ties) and weights = vals / (sum of the row's vals in
// rank order), each value with the unfused kernels' ops and order; vals and
// weights are stored when set.  x [T, H] f32 or bf16 at row stride x_rs
// (elements), W dense f32 [H, E], b f32 [E].
constexpr int kRouterMaxE = 64, kRouterMaxK = 16;
struct RouterArgs {
  const void* x;
  int x_bf16;
  int64_t x_rs;
  const float *w, *b;
  int64_t T, H;
  int E, k;
  int32_t* ids;
  float *vals, *weights;
};
// H % 64 == 0, 4 <= E <= 64, E % 4 == 0, 1 <= k <= min(E, 16), 16-byte
// aligned x rows and W
bool moe_router_ok(const RouterArgs& a);
void launch_moe_router(const RouterArgs& a, hipStream_t stream);

// ---- classifier head (k_head.hip) -----------------------------------------------
// ids[r] = argmax_j softmax(x[r] W + b)[j] over fp32 rows in one launch,
// each value with the unfused kernels' ops and order; the probabilities are
// also stored when `probs` is set.  x rows of K at row stride x_rs, W dense
// [K, N].
struct HeadArgs {
  const float* x;
  int64_t x_rs;
  const float *w, *b;
  int64_t M, K, N;
  float* probs;
  int32_t* ids;
};
// K % 4 == 0, K rounded up to 16 <= 1024, N <= 64, (K rounded up to 16) N
// <= 8192, 16-byte aligned x rows
bool class_head_ok(const HeadArgs& a);
void launch_class_head(const HeadArgs& a, hipStream_t stream);

// topK over the last dim of dense f32 [rows, cols]: vals / idx [rows, k],
// ranked larger-first (smaller-first when !largest), NaN last, ties to the
// lower column.  1 <= k <= 64, k <= cols <= kTopkMaxCols.
constexpr int64_t kTopkMaxCols = 4096;
struct TopkArgs {
  const float* x;
  float* vals;
  int32_t* idx;
  int64_t rows, cols;
  int k;
  int largest;
};
void launch_topk(const TopkArgs& g, hipStream_t stream);

// Row sort over the last dim (stablehlo.sort with a one-compare comparator,
// src/rew/ops/sort.nim:13-33): every operand is permuted by the order of
// the key operand; ascending (LT/LE) or descending (GT/GE), ties and NaN
// keys keep their original order, NaN keys rank after every number, -0 and
// +0 compare equal.  Keys: bool, 8/16/32-bit integers, f16, bf16, f32.
constexpr int kSortMaxOps = 4;
constexpr int64_t kSortMaxCols = 8192;
struct SortArgs {
  const void* key;
  int key_dt;
  int descending;
  int n_ops;
  const void* in[kSortMaxOps];
  void* out[kSortMaxOps];
  int esize[kSortMaxOps];   // 1, 2, 4 or 8 bytes
  int64_t rows, cols;
};
void launch_sort(const SortArgs& g, hipStream_t stream);

// ---- routed MoE (k_moe.hip) ------------------------------------------------------
constexpr int kMoeMaxK = 16;  // experts per token the combine handles
constexpr int kMoeMaxMembers = 1536;  // routed experts per call (placement LDS: 36 n bytes)
// Token placement for one group of routed experts ("members").
struct MoeRouteArgs {
  const int32_t* topi;       // [T, k] expert ids
  const float* topw;         // [T, k] gate weights
  int64_t T;
  int k;
  int E;                     // router width: ids are in [0, E)
  const int32_t* member_of;  // [E] member index or -1 (device)
  const int32_t* members;    // [n_members] expert id (device)
  int n_members;
  int32_t* off;              // [n_members + 1] packed row offsets (out)
  int32_t* mt_start;         // [n_members + 1] tile starts, group_tiles each (out)
  int32_t* perm;             // [T * k] packed row -> token (out)
  int32_t* ord_slot;         // [T, k] the token's packed rows in chain order, then -1 (out)
  float* ord_w;              // [T, k] their gate weights (out)
  int32_t* blk_cnt;          // [ceil(T / kMoeRouteBlock) * n_members] working counts
  // groups of all T tokens after the members (shared experts): off and
  // mt_start gain n_shared entries, perm rows T k + s T + t = t
  int n_shared;
};
constexpr int kMoeRouteBlock = 256;  // tokens per routing workgroup
int launch_moe_route(const MoeRouteArgs& a, hipStream_t stream);  // returns the launches

// out[t, :] = prev[t, :], then out = bf16(out + prev[s prev_sb + t, :]) for
// s = 1 .. n_prev - 1 (the shared experts' running sum), then, for token
// t's routed members in chain order, out = bf16(out + bf16(f32(y[slot, :]) *
// w)); bf16 rows, H % 8 == 0.
struct MoeCombineArgs {
  const uint16_t* prev;
  int64_t prev_rs;           // row stride of prev (elements)
  int n_prev = 1;            // prev rows folded per token
  int64_t prev_sb = 0;       // elements from one folded prev row set to the next
  const uint16_t* y;         // [T * k, H] packed expert outputs
  const int32_t* ord_slot;   // [T, k] from the placement
  const float* ord_w;        // [T, k]
  int64_t T, H;
  int k;
  uint16_t* out;             // dense [T, H]
};
void launch_moe_combine(const MoeCombineArgs& a, hipStream_t stream);

// The routed experts of rew's DeepSeekMoE.forward
// (src/rew/models/deepseek.nim:122-145) over dense bf16 rows:
//   out[t] = start[t] + sum over token t's routed experts e, in chain order,
//            of bf16(f32(down_e(SwiGLU_e(x[t]))) * w[t, e]),
// rounded to bf16 after every add -- the dense op sequence's arithmetic on
// the only rows where it is non-zero.  Expert `i` of the chain has id
// expert[i] in [0, E) and weights ptr[j][i] (device pointers, in the order
// gate W [H, I], up W [H, I], gate bias [I], up bias [I], down W [I, H],
// down bias [H]; W dense row-major).  `expert` and the six tables are host
// arrays of n entries.  Scratch: routed_ffn_scratch_bytes() of device
// memory, 256-byte aligned, that no other work uses meanwhile.
// With n_shared > 0 the shared experts come first and `start` is theirs:
//   start = bf16(... bf16(S_0(x) + S_1(x)) ... + S_{n_shared-1}(x)),
// S_s(x) = down_s(SwiGLU_s(x)) with the weights sptr[j][s] (same order as
// ptr); their SwiGLU GEMMs run in the routed experts' grouped launch as
// groups of all T rows, their down GEMMs as ordinary GEMMs with the bias
// and (after the first) residual epilogues, exactly the separate launches'
// arithmetic; `start` is then not read.
struct RoutedFfn {
  const void* x = nullptr;       // [T, H] bf16, rows x_rs apart
  int64_t x_rs = 0;
  const void* start = nullptr;   // [T, H] bf16: the sum before the routed experts
  int64_t start_rs = 0;
  const int32_t* topi = nullptr;  // [T, k] expert ids
  const float* topw = nullptr;    // [T, k] routing weights
  int64_t T = 0, H = 0, I = 0;
  int k = 0, E = 0, n = 0;
  const int32_t* expert = nullptr;
  const void* const* ptr[6] = {};
  int n_shared = 0;
  const void* const* sptr[6] = {};
  void* out = nullptr;           // [T, H] bf16, dense
};
// Throws Error(REW_MI355X_ERR_INVALID) naming the first argument the
// kernels cannot take.
void routed_ffn_check(const RoutedFfn& a);
size_t routed_ffn_scratch_bytes(const RoutedFfn& a);

// ---- fused attention (k_attn.hip) ---------------------------------------------
// out[b,h,i,:] = sum_j softmax_j(bf16(q[b,h,i,:].k[b,hk,j,:]) * scale + mask(i,j))
//                * v[b,hk,j,:],  hk = h / (H / Hkv); bf16 operands, d contiguous.
// mask(i, j) = cmp(i, j) ? mask_true : mask_false when `mask` is set.
struct FlashArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int B, H, Hkv, Sq, Sk, D;
  int64_t q_sb, q_sh, q_ss;  // strides in elements (b, head, position)
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  float scale;
  int round_scores;  // scores are rounded to bf16 before the fp32 scale / mask
  int mask;          // additive two-valued mask present
  int cmp;           // vm::Cmp direction of the predicate cmp(i, j)
  float mask_true, mask_false;
  int skip;          // key tiles masked everywhere may be skipped (exact)
  int heavy_last;    // the last query tiles carry the most keys
};
bool flash_supported(const FlashArgs& a);
// Fills the SwiGLU epilogue's table of x * logistic(x) over all bf16 x on
// the current device (once per context, before any GEMM).
void init_silu_table(hipStream_t stream);
// Profile name of the kernel launch_flash runs for `a`.
const char* flash_variant(const FlashArgs& a);

// ---- row composites (k_rows.hip) ----------------------------------------------
// rmsNorm over rows of n contiguous elements (x row stride x_rs elements):
// y[r, j] = gamma[j] * (x[r, j] / sqrt(sum_j x^2 / divisor + eps)).
struct RowNormArgs {
  const void* x;
  int x_dt;           // bf16 or f32 (converted to f32 on load)
  int64_t rows, n, x_rs;
  const float* gamma;
  float eps, divisor;
  void* y;            // dense [rows, n]
  int y_dt;           // bf16 or f32
  // gather form (an embedding lookup feeding the norm): source row r is row
  // ids[r] of x, clamped into [0, x_rows) like torchIndexSelect's gather,
  // and every gathered row is also stored to xout (dense [rows, n], x's
  // dtype); ids == nullptr: row r of x
  const void* ids;
  int ids_dt;
  int64_t x_rows;
  void* xout;
  // layer != 0: rew's LayerNorm (src/rew/nn/norm.nim:41-84) instead, op by
  // op in fp32:  m = sum_j x_j / divisor;  c_j = x_j - m;
  // v = sum_j c_j * c_j / divisor2;  y_j = gamma_j * (c_j * rsqrt(v + eps)) + beta_j
  int layer;
  const float* beta;
  float divisor2;
};
void launch_rmsnorm_rows(const RowNormArgs& a, hipStream_t stream);
// Whether launch_rmsnorm_rows runs the gather form of `a` (16-byte rows).
bool rmsnorm_gather_ok(const RowNormArgs& a);

// softmax over rows of n contiguous f32 (x row stride x_rs elements):
// m = max_j x, e_j = exp(x_j - m), s = sum_j e_j, y = e / s (dense f32).
// The sum runs in the order of the compiled row reduction, so y equals the
// reduceMax / sub / exp / reduceSum / divide sequence bit for bit.
struct SoftmaxArgs {
  const float* x;
  int64_t rows, n, x_rs;
  float* y;
};
// n < 128 (a thread per row) or n % 4 == 0, n <= kSoftmaxMaxCols, 16-byte
// aligned rows (a wave per row, the row held in registers)
constexpr int64_t kSoftmaxMaxCols = 8192;
bool softmax_rows_ok(const SoftmaxArgs& a);
void launch_softmax_rows(const SoftmaxArgs& a, hipStream_t stream);

// applyRotate on adjacent pairs over a [d0, d1, S, 2*half] index space; x,
// cos and sin are read through strided views (cos / sin indexed by pair i),
// y is dense.  half % 4 == 0 and d0*d1*S*half/4 < 2^31.
struct RopeArgs {
  const void* x;
  int x_dt;
  int64_t d0, d1, S, half;
  int64_t x_s0, x_s1, x_ss, x_sd;
  const float* cos;
  int64_t c_s0, c_s1, c_ss, c_si;
  const float* sin;
  int64_t s_s0, s_s1, s_ss, s_si;
  void* y;
  int y_dt;
  vm::FastDiv fd_g4, fd_s, fd_d1;  // divisors half/4, S, d1
};
void launch_rope(const RopeArgs& a, hipStream_t stream);
void launch_flash(const FlashArgs& a, hipStream_t stream);

}  // namespace rew
