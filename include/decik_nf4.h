/*
 * decik_nf4 — C ABI of the MI355X (gfx950) NF4 quantized-linear path.
 *
 * Every pointer is a device pointer (memory owned by the caller, e.g. PyTorch), except the
 * descriptor arrays themselves, which live in host memory and are copied into the kernel
 * arguments. fp16 tensors are passed as uint16_t (IEEE binary16 bit patterns). `stream` is a
 * hipStream_t (NULL = the default stream). Every entry point returns 0 on success and a
 * non-zero code on error; dk_last_error() then describes the error (per calling thread).
 * The library never allocates device memory: split-K workspaces are passed in.
 * The fused linear entries (forward, GLU forward, RoPE forward, input gradient with or without
 * the SwiGLU epilogue) accept m = 0 token rows: the shapes and descriptors are still checked,
 * nothing is launched, and the activation / output pointers may then be NULL.
 *
 * Reference interfaces replaced (tokha-t/decik, Python + Triton):
 *   dk_nf4_dequant / dk_nf4_dequant_batched  <- skc_nf4_dequant_kernel + dequantize_nf4
 *                                               (solution/nf4.py:27-48, 66-85)
 *   dk_nf4_block_scales                       <- the scale step of skc_nf4_dequant_kernel
 *                                               (solution/nf4.py:37-43)
 *   dk_nf4_linear_fwd                         <- NF4Linear.forward = dequantize_nf4 + F.linear
 *                                               (solution/nf4.py:93-96; solution/mlp.py:28-39),
 *                                               with peft's LoRA term added in the epilogue
 *                                               (solution/attn.py:225-228, 344-346)
 *   dk_nf4_linear_bwd                         <- NF4Linear.backward = dequantize_nf4 + matmul
 *                                               (solution/nf4.py:99-104); the summed input
 *                                               gradients of RecomputedMLP (solution/mlp.py:106-109)
 *                                               and of the LoRA branch (solution/attn.py:257)
 *   dk_nf4_linear_rope_fwd                    <- the q/k/v projections + FusedQKRope's forward
 *                                               (solution/attn.py:27-66, 396-418)
 *   dk_nf4_glu_fwd                            <- gate and up projections + _swiglu_fwd of the
 *                                               Qwen2 MLP forward (solution/mlp.py:69-71)
 *   dk_nf4_linear_bwd_swiglu                  <- matmul(g16, w_down) + _swiglu_bwd of the MLP
 *                                               backward (solution/mlp.py:95, 104)
 *   dk_lora_down / dk_lora_bwd                <- the rank-r products of LoRAPairFromNorm
 *                                               (solution/attn.py:225-227, 251-257)
 *   dk_lora_down_group / dk_lora_bwd_group    <- the same products of LoRAPairFromNorm's q and v
 *                                               branches, one launch for both (attn.py:206-273)
 *   dk_lora_down_dropout / dk_lora_bwd_dropout <- the same with skc_lora_inputs_kernel fused in
 *     + dk_linear_bwd_group.lora_keep            and skc_lora_input_grad_kernel in the input-
 *                                               gradient GEMM (solution/attn.py:153-180, 206-273)
 *   dk_lora_keep_pack                         <- skc_keep_pack_kernel / pack_keep
 *                                               (solution/attn.py:129-144, 195-203)
 *   dk_lora_dropout_inputs                    <- skc_lora_inputs_kernel / _lora_inputs
 *                                               (solution/attn.py:153-165, 183-192)
 *   dk_lora_input_grad                        <- skc_lora_input_grad_kernel (solution/attn.py:168-180)
 *   dk_lora_up                                <- grad_u.mm(a16) of LoRAPairFromNorm.backward
 *                                               (solution/attn.py:257)
 *   dk_rope_qk_fwd / dk_rope_qk_bwd           <- skc_rope_fwd_kernel / skc_rope_bwd_kernel and
 *                                               FusedQKRope (solution/attn.py:27-126)
 *   dk_swiglu_fwd / dk_swiglu_bwd             <- example_swiglu_fwd/bwd_kernel
 *                                               (solution/swiglu.py:15-37)
 */
#ifndef DECIK_NF4_H
#define DECIK_NF4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DK_MAX_GROUPS 4

/* A bitsandbytes nf4 weight: Params4bit bytes + QuantState fields read by the reference
 * (solution/nf4.py:54-58, 70-79). Weight shape [n, k] row-major; flat element index
 * i = row * k + col; block = i / blocksize; group = block / blocksize2. */
typedef struct dk_nf4_weight {
    const uint8_t* packed;  /* [n*k/2] bytes, element 2j in the high nibble of byte j   */
    const void* absmax;     /* nested: uint8 codes [n_blocks]; plain: fp32 [n_blocks]   */
    const float* absmax2;   /* nested: fp32 [ceil(n_blocks / blocksize2)]; else NULL   */
    const float* code2;     /* nested: fp32 [256] (state2.code); else NULL              */
    const float* offset;    /* nested: fp32 scalar (QuantState.offset); else NULL       */
    const float* code;      /* fp32 [16] NF4 code book (QuantState.code)                */
    int64_t n, k;           /* weight shape                                             */
    int32_t blocksize;      /* QuantState.blocksize (even, >= 2)                        */
    int32_t blocksize2;     /* state2.blocksize (nested only)                           */
    int32_t nested;         /* QuantState.nested                                        */
    int32_t reserved;
} dk_nf4_weight;

/* One weight of a forward launch. Y[r, c] = sum_j X[r, j] W[c, j] + bias[c]
 *                                        + lora_scale * sum_t U[r, t] B[c, t]
 * (U = X.A^T from dk_lora_down, fp16 [m, rank]; B fp16 [n, rank]). */
typedef struct dk_linear_fwd_group {
    dk_nf4_weight w;
    const uint16_t* bias;    /* fp16 [n] or NULL (16-byte aligned)         */
    const uint16_t* lora_u;  /* fp16 [m, rank] or NULL (no LoRA term)      */
    const uint16_t* lora_b;  /* fp16 [n, rank]; U and B 16-byte aligned    */
    float lora_scale;
    int32_t reserved;
    uint16_t* y;             /* fp16 output, row stride ldy (elements)    */
    int64_t ldy;
} dk_linear_fwd_group;

/* One weight of a backward launch. Its contribution to dX[r, j] is
 *   sum_c dY[r, c] W[c, j] + sum_t GU[r, t] A[t, j]
 * (GU = lora_scale * dY.B from dk_lora_bwd, fp16 [m, rank]; A fp16 [rank, k]). With lora_keep
 * (the LoRA branch's input went through dropout, LoRAPairFromNorm's packed masks,
 * solution/attn.py:168-180, 251-266) the LoRA part is instead
 *   (fp16(sum_t GU[r, t] A[t, j]) * keep[r, j]) * lora_keep_scale     (fp32)
 * with keep[r, j] = bit j % 8 of byte r * (k / 8) + j / 8 of lora_keep (dk_lora_keep_pack). */
typedef struct dk_linear_bwd_group {
    dk_nf4_weight w;
    const uint16_t* dy;      /* fp16 [m, n], row stride lddy              */
    int64_t lddy;
    const uint16_t* lora_gu; /* fp16 [m, rank] or NULL                    */
    const uint16_t* lora_a;  /* fp16 [rank, k]                            */
    const uint8_t* lora_keep; /* packed keep bits [m, k / 8] or NULL      */
    float lora_keep_scale;   /* 1 / (1 - p)                               */
    int32_t reserved;
} dk_linear_bwd_group;

/* Standalone dequantization: out = fp16 [n, k], bit-identical to the reference kernel
 * (code[nibble] * scale in fp32, nested scale = code2[q] * absmax2 + offset with two
 * roundings, round to nearest even). */
int dk_nf4_dequant(const dk_nf4_weight* w, uint16_t* out, void* stream);

/* The same for `count` weights in one launch (out[i] receives weight i). */
int dk_nf4_dequant_batched(const dk_nf4_weight* ws, uint16_t* const* outs, int count,
                           void* stream);

/* fp32 scale of every block, scales[ceil(n*k / blocksize)]: the scale computation of
 * skc_nf4_dequant_kernel (solution/nf4.py:37-43) on its own, with the same two roundings. A
 * weight described as plain (nested = 0) with absmax = these scales dequantizes to the same
 * bits; the fused GEMMs run faster on it (one fp32 load per block instead of the code2 /
 * absmax2 chain), so a caller may compute it once per frozen weight and reuse it. */
int dk_nf4_block_scales(const dk_nf4_weight* w, float* scales, void* stream);

/* Bytes of workspace dk_nf4_linear_fwd needs for these shapes (0 if none), whatever the block
 * sizes, statistics form and LoRA terms of the call: the fp32 partial sums of a split
 * contraction. Its contents need not be initialised and are dead after the call. Calls that run
 * concurrently (different streams) need different workspaces. */
int64_t dk_nf4_linear_fwd_workspace(int64_t m, int64_t k, const int64_t* ns, int ngroups);

/* Fused dequant x fp16 GEMM, forward, for up to DK_MAX_GROUPS weights that share X
 * (fp16 [m, k], row stride ldx). fp32 accumulation, one fp16 rounding per output.
 * Shapes: k % 32 == 0, every weight's n % 8 == 0 (outputs move in 8-column chunks), blocksize a
 * power of two >= 32 dividing 64 * k; x, y, bias, packed 16-byte aligned, ldx / ldy % 8 == 0.
 * Anything else returns an error (the Python layer sends such weights to dequant + F.linear). */
int dk_nf4_linear_fwd(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                      const dk_linear_fwd_group* groups, int ngroups, int lora_rank,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* dk_nf4_linear_fwd with RoPE and the head-major store of the attention inputs in its epilogue
 * (the q/k projections followed by skc_rope_fwd_kernel / FusedQKRope, solution/attn.py:27-66,
 * 396-418): for each group g whose bit is set in rope_mask, the projection output, rounded to fp16,
 * is rotated per token as x cos + rotate_half(x) sin in fp32 (the reference's order, no fused
 * multiply-add) and stored fp16 head-major to rope_out[g] [n_g / head_dim, m, head_dim]; its
 * groups[g].y is not used. Other groups are stored as by dk_nf4_linear_fwd. cos, sin: fp32
 * [m, head_dim]; head_dim % 16 == 0; n_g % head_dim == 0. The contraction is always split (the
 * rotation runs in the split-K reduction), so k >= 128 and a workspace of
 * dk_nf4_linear_rope_fwd_workspace bytes is needed. The q/k/v projection of a Qwen2 layer is one
 * call: groups q, k, v with rope_mask 3. */
int64_t dk_nf4_linear_rope_fwd_workspace(int64_t m, int64_t k, const int64_t* ns, int ngroups);
int dk_nf4_linear_rope_fwd(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                           const dk_linear_fwd_group* groups, int ngroups, int lora_rank, const float* cos,
                           const float* sin, int head_dim, int rope_mask, uint16_t* const* rope_out,
                           void* workspace, int64_t workspace_bytes, void* stream);

/* Gate and up projections and SwiGLU in one launch: groups[0] = gate, groups[1] = up (one shape
 * [n, k]; bias and LoRA as in dk_nf4_linear_fwd), h = fp16(silu(gate) * up) [m, n] (row stride
 * ldh) from the fp16-rounded gate and up -- the same bits as dk_nf4_linear_fwd followed by
 * dk_swiglu_fwd. One launch when gate and up have the same statistics kind (both plain or both
 * nested, as bitsandbytes stores them), blocksize >= 64 and k % 64 == 0; then groups[i].y may be
 * NULL (not stored). Other weights run as the grouped launch then the SwiGLU kernel and need both
 * y, with rows contiguous (ldy = ldh = n). No workspace. */
int dk_nf4_glu_fwd(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                   const dk_linear_fwd_group* groups, int lora_rank, uint16_t* h, int64_t ldh,
                   void* stream);

/* As dk_nf4_linear_fwd_workspace, for dk_nf4_linear_bwd. */
int64_t dk_nf4_linear_bwd_workspace(int64_t m, int64_t k, const int64_t* ns, int ngroups);

/* Fused dequant x fp16 GEMM, input gradient: dX = sum over groups of dY_g.W_g (+ GU_g.A_g),
 * accumulated in fp32 across all groups and rounded once. dx is fp16 (dx_fp32 = 0) or fp32
 * (dx_fp32 = 1), row stride lddx. Shapes as for dk_nf4_linear_fwd (k % 32 == 0, n % 8 == 0). */
int dk_nf4_linear_bwd(const dk_linear_bwd_group* groups, int ngroups, int64_t m, int64_t k,
                      void* dx, int64_t lddx, int dx_fp32, int lora_rank, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* No counterpart in the reference: dk_nf4_linear_bwd for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results as dk_nf4_linear_bwd, without the workspace: the split-K partial
 * sums live in a static device array of DK_NOALLOC_SCRATCH_BYTES per GPU, held from the first
 * call on that GPU until the process ends. Launch plans are capped so that their partials fit
 * (fewer splits, or none), so every shape dk_nf4_linear_bwd takes runs here; when the allocating
 * entry's plan fits, both run the same plan and give the same bits. Nothing carries over
 * between calls. Calls and graph replays on one GPU share the array: calls that overlap in time
 * on one GPU (different streams, concurrent replays) race and must be serialised by the caller.
 * Allocates nothing (no hipMalloc, hipFree or allocating library routine). */
#define DK_NOALLOC_SCRATCH_BYTES (64ll << 20)
int dk_nf4_linear_bwd_noalloc(const dk_linear_bwd_group* groups, int ngroups, int64_t m, int64_t k,
                              void* dx, int64_t lddx, int dx_fp32, int lora_rank, void* stream);

/* Input gradient of one weight (the MLP's down projection, group->w [n, k]) with the SwiGLU
 * backward in its epilogue: G = fp16(dY . W) [m, k] is never stored; dgate =
 * fp16(G up s (1 + gate (1 - s))), dup = fp16(G gate s), s = sigmoid(gate) -- the same bits as
 * dk_nf4_linear_bwd followed by dk_swiglu_bwd. gate, up fp16 [m, k] (row stride ldgu); dgate,
 * dup fp16 [m, k] (row stride ldd), which may alias gate and up. No workspace. */
int dk_nf4_linear_bwd_swiglu(const dk_linear_bwd_group* group, int64_t m, int64_t k, int lora_rank,
                             const uint16_t* gate, const uint16_t* up, int64_t ldgu, uint16_t* dgate,
                             uint16_t* dup, int64_t ldd, void* stream);

/* U = fp16(X . A^T): X fp16 [m, k] (row stride ldx), A fp16 [rank, k], U fp16 [m, rank]. */
int dk_lora_down(const uint16_t* x, int64_t m, int64_t k, int64_t ldx, const uint16_t* a,
                 int rank, uint16_t* u, void* stream);

/* LoRA weight and input-branch gradients for out = scale * (U . B^T), U = X . A^T:
 *   GU = fp16(scale * dY . B)  [m, rank]
 *   dB = scale * dY^T . U      fp32 [n, rank]
 *   dA = GU^T . X              fp32 [rank, k]
 * dY fp16 [m, n] (row stride lddy; n and lddy multiples of 8), U fp16 [m, rank], X fp16 [m, k]
 * (row stride ldx), B fp16 [n, rank]; da or db may be NULL (not computed). Fixed summation order:
 * the same bits on every call. The input gradient GU . A is added by dk_nf4_linear_bwd. */
int dk_lora_bwd(const uint16_t* dy, int64_t lddy, const uint16_t* u, const uint16_t* x,
                int64_t ldx, const uint16_t* b, int64_t m, int64_t n, int64_t k, int rank,
                float scale, uint16_t* gu, float* da, float* db, void* stream);

/* dk_lora_down and dk_lora_bwd with the branch's input X given as the norm output the reference
 * feeds LoRAPairFromNorm (solution/attn.py:153-165, 219-228, 241-257): x fp16 (x_fp32 = 0) or
 * fp32 [m, k] (row stride ldx, 16-byte aligned), and optionally through dropout: X = fp16(x *
 * (keep * keep_scale)) in fp32 (skc_lora_inputs_kernel's rounding), keep[r, j] = bit j % 8 of
 * byte r * (k / 8) + j / 8 of keep_bits (dk_lora_keep_pack), keep_scale a device fp32 scalar
 * (1 / (1 - p)). keep_bits NULL: X = fp16(x). The dropped-out input is rebuilt in registers and
 * never stored; the backward GEMM applies the same mask to the branch's input gradient
 * (dk_linear_bwd_group.lora_keep). */
int dk_lora_down_dropout(const void* x, int x_fp32, int64_t m, int64_t k, int64_t ldx,
                         const uint8_t* keep_bits, const float* keep_scale, const uint16_t* a, int rank,
                         uint16_t* u, void* stream);
int dk_lora_bwd_dropout(const uint16_t* dy, int64_t lddy, const uint16_t* u, const void* x, int x_fp32,
                        int64_t ldx, const uint8_t* keep_bits, const float* keep_scale, const uint16_t* b,
                        int64_t m, int64_t n, int64_t k, int rank, float scale, uint16_t* gu, float* da,
                        float* db, void* stream);

/* One LoRA branch (one adapter: q or v) of a grouped call. */
typedef struct dk_lora_branch {
    const void* x;            /* the branch input, fp16 (x_fp32 = 0) or fp32 [m, k], row stride ldx */
    const uint8_t* keep_bits; /* NULL, or packed dropout keep bits [m, k / 8] (as above)        */
    const float* keep_scale;  /* device fp32 scalar 1 / (1 - p) with keep_bits                 */
    const uint16_t* a;        /* A fp16 [rank, k]                                               */
    uint16_t* u;              /* U fp16 [m, rank]: written by _down, read by _bwd               */
    const uint16_t* dy;       /* _bwd: dY fp16 [m, n], row stride lddy                          */
    const uint16_t* b;        /* _bwd: B fp16 [n, rank]                                         */
    uint16_t* gu;             /* _bwd: GU fp16 [m, rank] out                                    */
    float* da;                /* _bwd: dA fp32 [rank, k] out, or NULL                           */
    float* db;                /* _bwd: dB fp32 [n, rank] out, or NULL                           */
    int64_t ldx, lddy, n;
    float scale;              /* _bwd: the LoRA scaling s                                       */
    int32_t x_fp32;
} dk_lora_branch;

/* dk_lora_down_dropout / dk_lora_bwd_dropout for 1..4 branches that share m, k and the rank (the
 * q and v adapters of one layer, LoRAPairFromNorm's two branches, solution/attn.py:206-273): each
 * product of every branch in one launch (one per kind of input -- fp16 / fp32, with / without
 * dropout -- where the branches' kinds differ) instead of one launch per branch, with the same
 * bits as the per-branch calls. _down reads x, keep_bits, keep_scale, a and writes u; _bwd reads
 * every field but a and writes gu, da, db. */
int dk_lora_down_group(const dk_lora_branch* branches, int nbranches, int64_t m, int64_t k, int rank,
                       void* stream);
int dk_lora_bwd_group(const dk_lora_branch* branches, int nbranches, int64_t m, int64_t k, int rank,
                      void* stream);

/* LoRA dropout (the packed-mask path of LoRAPairFromNorm). Masks are bool bytes (0/1), rows x width
 * row-major, width % 8 == 0; bits are [rows, width / 8]. */

/* bits_q[r, c / 8] bit (c % 8) = keep_q[r, c], the same for v (keep_* 8-byte aligned). */
int dk_lora_keep_pack(const uint8_t* keep_q, const uint8_t* keep_v, uint8_t* bits_q, uint8_t* bits_v,
                      int64_t rows, int64_t width, void* stream);

/* xq = fp16(x * (keep_q * scale_q)), xv = fp16(x * (keep_v * scale_v)) in fp32; x fp16 (x_fp32 = 0)
 * or fp32 [rows, width]; scale_q, scale_v: device fp32 scalars (the kept value 1 / (1 - p)). */
int dk_lora_dropout_inputs(const void* x, int x_fp32, const uint8_t* bits_q, const uint8_t* bits_v,
                           const float* scale_q, const float* scale_v, uint16_t* xq, uint16_t* xv,
                           int64_t rows, int64_t width, void* stream);

/* out = (fp32(gq) * keep_q) * scale_q + (fp32(gv) * keep_v) * scale_v, fp32 [rows, width]: the input
 * gradient of both branches through their dropout. */
int dk_lora_input_grad(const uint16_t* gq, const uint16_t* gv, const uint8_t* bits_q, const uint8_t* bits_v,
                       float scale_q, float scale_v, float* out, int64_t rows, int64_t width, void* stream);

/* A branch's input gradient before its dropout mask: out = fp16(GU . A) [m, k], GU fp16 [m, rank],
 * A fp16 [rank, k] (rank 16 or 32, k % 8 == 0). */
int dk_lora_up(const uint16_t* gu, const uint16_t* a, int rank, uint16_t* out, int64_t m, int64_t k, void* stream);

/* RoPE of the attention inputs, q and k in one launch: q = fp32(q_base) + fp32(q_lora) (q_lora may
 * be NULL: no addition), out = q * cos + rotate_half(q) * sin in fp32, stored fp16 head-major
 * q_out [n_heads, n_tok, head_dim], k_out [n_kv_heads, n_tok, head_dim]; k likewise without LoRA.
 * q_base / q_lora / k: fp16 token-major with row strides ldq / ldl / ldk; cos, sin: fp32
 * [n_tok, head_dim]; head_dim % 16 == 0. */
int dk_rope_qk_fwd(const uint16_t* q_base, const uint16_t* q_lora, int64_t ldq, int64_t ldl, const uint16_t* k,
                   int64_t ldk, const float* cos, const float* sin, uint16_t* q_out, uint16_t* k_out, int64_t n_tok,
                   int n_heads, int n_kv_heads, int head_dim, void* stream);

/* Its transpose: d = g * cos + rotate_half^T(g * sin) in fp32, rounded to fp16 once; grad_q / grad_k
 * head-major fp16, dq / dk token-major with row strides lddq / lddk. */
int dk_rope_qk_bwd(const uint16_t* grad_q, const uint16_t* grad_k, const float* cos, const float* sin, uint16_t* dq,
                   int64_t lddq, uint16_t* dk, int64_t lddk, int64_t n_tok, int n_heads, int n_kv_heads, int head_dim,
                   void* stream);

/* out = fp16(silu(gate) * up), computed in fp32 (n elements). */
int dk_swiglu_fwd(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n,
                  void* stream);

/* dgate = fp16(G up s (1 + gate (1 - s))), dup = fp16(G gate s), s = sigmoid(gate).
 * dgate/dup may alias gate/up (every element is read before it is written). */
int dk_swiglu_bwd(const uint16_t* grad, const uint16_t* gate, const uint16_t* up,
                  uint16_t* dgate, uint16_t* dup, int64_t n, void* stream);

/* Diagnostic, no counterpart in the reference: the launch plan that dk_nf4_linear_fwd
 * (backward = 0) or dk_nf4_linear_bwd (backward = 1) chooses for these shapes, for reports and
 * tuning. flags: DK_PLAN_GLU (forward: the fused GLU mode of dk_nf4_glu_fwd; backward: the SwiGLU
 * epilogue of dk_nf4_linear_bwd_swiglu), DK_PLAN_LORA (some group has LoRA terms),
 * DK_PLAN_NO_SPLIT (a single pass), DK_PLAN_NESTED (with DK_PLAN_GLU, forward: the weights carry
 * nested statistics), DK_PLAN_PARTS (out holds 6 values: out[4] = GEMM launches of the call, 2
 * when an input gradient whose tiles overrun whole rounds of CUs runs its left-over columns as a
 * second launch, and out[5] = that launch's contraction splits; out[0..3] then describe the
 * first launch). blocksize: the largest block size of the groups' weights.
 * out[0] = 32-token row blocks per tile, out[1] = waves per work-group, out[2] = contraction
 * splits, out[3] = kernel (0 nf4_fwd_kernel, 1 nf4_fwd8_kernel, 2 no longer returned (an
 * earlier input-gradient kernel), 3 nf4_bwd8_kernel, 4 nf4_gemv_kernel (forward launches of one
 * token row, two with fewer than 2^25 weights and k <= 12288 (any k up to 2^24 weights), 3-4
 * with at most 2^24 weights, 5-8 with fewer than 2^23 weights
 * and 8 k <= 32768, without LoRA terms or the GLU epilogue), 5
 * nf4_skinny_kernel (such launches of up to 32 token rows otherwise, but past 16 rows not for
 * weights of more 64-row groups than the device has CUs; out[2] is then its contraction splits); DECIK_SMALL_M = gemv / skinny picks one
 * of the two where both may run). Host-only (no GPU call);
 * honours DECIK_FWD_PLAN / DECIK_BWD_PLAN / DECIK_SMALL_M like the launches. Returns 0, or nonzero
 * with dk_last_error() on bad arguments. */
#define DK_PLAN_GLU 1
#define DK_PLAN_LORA 2
#define DK_PLAN_NO_SPLIT 4
#define DK_PLAN_NESTED 8
#define DK_PLAN_PARTS 16
int dk_nf4_linear_plan(int backward, int64_t m, int64_t k, const int64_t* ns, int ngroups, int flags,
                       int blocksize, int32_t* out);

/* Diagnostic, no counterpart in the reference: the device's dense fp16 MFMA rate, for reporting
 * the GEMM kernels against a measured ceiling. Runs work_groups x 8 waves, each `iters` rounds of
 * 8 v_mfma_f32_32x32x16_f16 on register operands (work_groups * 8 * iters * 8 * 32768 flops);
 * out: work_groups * 512 floats (written, values meaningless). Allocates nothing. */
int dk_probe_mfma_f16(int64_t work_groups, int32_t iters, float* out, void* stream);

/* Diagnostic, no counterpart in the reference: this device's HBM streaming rate, with the access
 * pattern of the dequantization kernel (16-byte lanes, every chunk of a thread in flight at
 * once). mode 0: read `bytes` of src (sums: one float per 16 KB of src, written only to keep the
 * loads, in practice never); 1: write `bytes` of dst; 2: copy src to dst; + 4: plain instead of
 * non-temporal stores; + 8: plain instead of non-temporal loads; + 16 / + 32: 8 / 16 chunks per
 * thread instead of 4. bytes % 16 == 0, src and dst 16-byte aligned. Allocates nothing. */
int dk_probe_hbm(const void* src, void* dst, int64_t bytes, int mode, float* sums, void* stream);

/* Description of the last error on the calling thread ("" if none). */
const char* dk_last_error(void);

/* Library version (major * 10000 + minor * 100 + patch). */
int dk_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DECIK_NF4_H */
