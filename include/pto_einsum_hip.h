/*
 * pto_einsum_hip.h -- C ABI of the MI355X (gfx950) einsum backend.
 *
 * Two layers, both plain C (pointers, sizes, a void* hipStream_t):
 *
 *  1. Per-shape entry points.  Every JIT library the Python builder generates
 *     for one (equation, shapes, dtype) exports exactly the symbol set the
 *     reference binds through ctypes (reference builder.py:761-815; wrappers
 *     in templates.py:74-92, 111-129, 158-191).  T is `float` or `uint16_t`
 *     (IEEE half bits, the reference's ctypes c_uint16); outputs are float.
 *     Where the reference returns void, these return 0 or a pe_status code.
 *
 *  2. The core library (libpto_einsum_hip.so) the per-shape wrappers call:
 *     descriptor-driven launchers for the three kernel families (strided
 *     product, permutation copy, batched MFMA GEMM) and the plan executor.
 *
 * Streams: `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream);
 * NULL means the default stream.  All launches are asynchronous; nothing in
 * an exec path allocates, frees or synchronizes.
 */
#ifndef PTO_EINSUM_HIP_H
#define PTO_EINSUM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PE_MAX_DIMS 8

/* Status codes.  Positive values are hipError_t codes from the runtime. */
enum pe_status {
    PE_OK = 0,
    PE_ERR_INVALID = -1,     /* descriptor inconsistent (message: pe_last_error) */
    PE_ERR_BOUNDS = -2,      /* descriptor would address outside an operand */
    PE_ERR_UNSUPPORTED = -3, /* dtype / rank / layout the kernels do not cover */
    PE_ERR_WORKSPACE = -4    /* workspace missing or too small */
};

enum pe_dtype { PE_F32 = 0, PE_F16 = 1 };

/* Contraction-free product over a row-major float32 output:
 *   out[o] = (add_zero ? 0.0f + a*b : a*b),  a = (float)in0[sum_d o_d*a_stride[d]],
 *                                           b = (float)in1[sum_d o_d*b_stride[d]].
 * add_zero = 1 reproduces the reference CPU route's C=1 matmul accumulation
 * (cpu_einsum.h:71-76: accum = 0; accum += a*b), 0 its Hadamard multiply
 * (cpu_einsum.h:87-92).  Covers Hadamard, broadcast, outer and transposed
 * elementwise products. */
typedef struct pe_product_desc {
    int32_t dtype;
    int32_t add_zero;
    int32_t ndims;                      /* 0..PE_MAX_DIMS */
    int32_t _pad;
    int64_t shape[PE_MAX_DIMS];         /* output extents, outermost first */
    int64_t a_stride[PE_MAX_DIMS];      /* in0 element stride per output axis */
    int64_t b_stride[PE_MAX_DIMS];      /* in1 element stride per output axis */
    int64_t a_numel, b_numel;           /* operand extents, for bounds checks */
} pe_product_desc;

/* Permutation copy (bit-exact): dst is row-major over `shape`;
 *   dst[o] = src[sum_d o_d * src_stride[d]]
 * i.e. the reference's transfer_idx map with to_shape = shape and
 * perm_strides = src_stride (cpu_einsum.h:35-51). */
typedef struct pe_permute_desc {
    int32_t elem_bytes;                 /* 2 or 4 */
    int32_t ndims;
    int64_t shape[PE_MAX_DIMS];
    int64_t src_stride[PE_MAX_DIMS];
    int64_t src_numel;
} pe_permute_desc;

/* Batched strided GEMM with float32 accumulation:
 *   C[b,m,n] = sum_k (float)A[b,m,k] * (float)B[b,k,n]
 * with A at a_off(b) + m*a_ms + k*a_ks, B at b_off(b) + k*b_ks + n*b_ns and
 * C at c_off(b) + m*c_ms + n*c_ns, where x_off(b) decodes the flat batch
 * index over batch_shape (row-major) with the per-axis x_bstride. */
typedef struct pe_gemm_desc {
    int32_t dtype;
    int32_t nbatch;                     /* 0..PE_MAX_DIMS batch axes */
    int32_t split_k;                    /* 0 = choose; else number of K splits */
    int32_t tile;                       /* 0 = choose; 64 or 128 (square); 256 = 256x128
                                           (M >= N) or 128x256; 192 (float32 only) =
                                           192x128 (M >= N) or 128x192; 1 = the float16
                                           256x256 kernel; 2 = the short-K kernel (all of K
                                           resident in LDS: float16 K in (96, 128] on 64x128
                                           tiles, float32 K in (112, 128] on 128x128) */
    int64_t batch_shape[PE_MAX_DIMS];
    int64_t a_bstride[PE_MAX_DIMS], b_bstride[PE_MAX_DIMS], c_bstride[PE_MAX_DIMS];
    int64_t M, N, K;
    int64_t a_ms, a_ks, b_ks, b_ns, c_ms, c_ns;
    int64_t a_numel, b_numel, c_numel;
} pe_gemm_desc;

enum pe_route { PE_ROUTE_PRODUCT = 0, PE_ROUTE_GEMM = 1 };

/* A whole einsum: either one product launch, or
 *   [gather in0 -> ws] [gather in1 -> ws] GEMM [ws -> permute into out].
 * Workspace regions are byte offsets into the buffer run_einsum_setup returns. */
typedef struct pe_einsum_plan {
    int32_t route;
    int32_t gather0, gather1, scatter_out;  /* 1 = stage through workspace */
    pe_product_desc product;
    pe_permute_desc perm0, perm1, perm_out;
    pe_gemm_desc gemm;
    int64_t ws0_off, ws1_off, wsout_off, wsgemm_off;
    int64_t ws_bytes;                     /* total workspace bytes */
    /* Phase ablation for timing by subtraction (the reference's
     * EINSUM_PHASE_STOP, include/pto_einsum.h:17-29, builder.py:688-697):
     * bit 0 skips phase A (the operand gathers), bit 1 phase B (the GEMM with
     * its split reduction, or the product kernel), bit 2 phase C (the output
     * permutation).  Skipped phases launch nothing and leave what they would
     * write unwritten.  0 runs the whole plan.  The per-shape wrapper sets it
     * from EINSUM_PHASE_STOP = N (default 3): the phases after the N-th. */
    int32_t skip_phases;
    int32_t reserved;                     /* must be 0 */
} pe_einsum_plan;

/* ---- core library (libpto_einsum_hip.so) ---- */

/* Launchers: validate the descriptor on the host, then enqueue on `stream`. */
int pe_product(const pe_product_desc* d, const void* in0, const void* in1, float* out,
               void* stream);
int pe_permute(const pe_permute_desc* d, const void* src, void* dst, void* stream);
/* pe_gemm's workspace (0 when K is not split): the split-K partial sums,
 * nsplit x batches x M x N float32, summed in split order by a second
 * kernel. */
int64_t pe_gemm_workspace_bytes(const pe_gemm_desc* d);
int pe_gemm(const pe_gemm_desc* d, const void* a, const void* b, float* c, void* ws,
            int64_t ws_bytes, void* stream);
/* The tile and K split pe_gemm takes for these extents and strides, operand
 * pointers taken as 16-byte aligned (no counterpart in the reference; for
 * tests and tuning): info[0..3] = tile rows, tile columns, K splits, k per
 * split (256 x 256 for the large float16 kernel).  The split, and so the
 * workspace size, is the same for every operand layout. */
int pe_gemm_choice(const pe_gemm_desc* d, int64_t* info);

/* Fused linear-attention chain.  No single entry point of the reference
 * corresponds: it runs the chain as three einsums with float32 intermediates
 * (tests/test_llm_ops.py:81-107, benchmarks/complex/bench_linear_attention.py:62-94):
 *   A = einsum("tn,sn->ts", q, k); A = einsum("ts,ts->ts", A, m);
 *   out = einsum("ts,sp->tp", A, v).
 * This launches it as one kernel (plus a split reduction when the workspace
 * is used): out[t,p] = sum_s ((sum_n q[t,n] k[s,n]) * m[t,s]) * v[s,p], every
 * operand read as float32 (float16 up-cast exactly), the inner sum and the
 * mask product rounded to float32 as in the three-step chain.  Rows of q, k,
 * v and m are contiguous with the given row strides; out is [T][P] float32.
 * N <= 256 for float16 q/k, N <= 128 for float32.  The workspace holds split
 * partials and zero-padded copies of q / k / m when their rows are not whole
 * 16-byte (q, k) or 4-element (m) vectors; the size query assumes 16-byte
 * aligned base addresses (a misaligned base needs a padded copy too). */
typedef struct pe_linattn_desc {
    int32_t qk_dtype;                   /* element type of q and k */
    int32_t v_dtype;
    int32_t m_dtype;
    int32_t split;                      /* 0 = choose; else number of s splits */
    int64_t T, S, N, P;
    int64_t q_ts, k_ss, v_ss, m_ts;     /* row strides, in elements */
    int64_t q_numel, k_numel, v_numel, m_numel;
    int32_t precise;                    /* 1: P.V on float32 MFMAs; 0 (default): P and V split
                                           into bfloat16 hi + lo, P.V as three bf16 MFMA terms
                                           (products exact, float32 sums; each dropped term
                                           below 2^-16 |P||V|) */
    int32_t reserved;                   /* must be 0 */
} pe_linattn_desc;

int64_t pe_linear_attention_workspace_bytes(const pe_linattn_desc* d);
int pe_linear_attention(const pe_linattn_desc* d, const void* q, const void* k, const void* v,
                        const void* m, float* out, void* ws, int64_t ws_bytes, void* stream);

/* Sum over the solo axes of one einsum operand (an index found in that
 * operand only and not in the output).  No entry point of the reference
 * corresponds: it rejects such equations (builder.py:218-229); this is the
 * reduction stage its roadmap describes for them (IMPLEMENTATION.md:812-821,
 * "Option A"), reached from Python through einsum(..., reduce_solo_axes=True).
 *   dst[k] = sum over r of (float)src[sum_d k_d keep_stride[d] + sum_e r_e red_stride[e]]
 * with k the row-major index over keep_shape (dst contiguous float32) and r
 * over red_shape.  Order (a function of the shapes, of whether the reduced axes
 * form one stride-1 run, of 16-byte alignment and of the dtype -- never of the
 * device -- so deterministic), with (V, L, C) as pe_reduce_order reports: the
 * nterm terms of an output, row-major in r, form G = ceil(nterm / V) groups of V
 * consecutive terms; the groups are cut into C contiguous chunks (the first
 * G % C one group longer); in a chunk, lane l of L sums groups l, l + L, ...
 * term by term from +0; the L lane sums, then the C chunk sums, are combined by
 * a pairwise tree (for s = 1, 2, 4, ...: p[i] += p[i + s] for i a multiple of 2s
 * with i + s in range; the result is p[0]).  An empty reduced axis gives +0.
 * With C > 1 the call needs a workspace of pe_reduce_workspace_bytes(d) bytes
 * (ws, ws_bytes); otherwise ws may be null.
 * nred = 0 is a conversion to float32. */
typedef struct pe_reduce_desc {
    int32_t dtype;                      /* PE_F32 or PE_F16 */
    int32_t nkeep;                      /* 0..PE_MAX_DIMS */
    int32_t nred;                       /* 0..PE_MAX_DIMS */
    int32_t reserved;                   /* must be 0 */
    int64_t keep_shape[PE_MAX_DIMS], keep_stride[PE_MAX_DIMS];
    int64_t red_shape[PE_MAX_DIMS], red_stride[PE_MAX_DIMS];
    int64_t src_numel;
} pe_reduce_desc;

int pe_reduce_axes(const pe_reduce_desc* d, const void* src, float* dst, void* ws, int64_t ws_bytes,
                   void* stream);
/* Workspace bytes pe_reduce_axes needs for d at any source address (the larger
 * of the 16-byte-aligned and unaligned plans; 0 when C = 1 for both, or d is
 * invalid). */
int64_t pe_reduce_workspace_bytes(const pe_reduce_desc* d);
/* The (V, L, C) of the summation order above for d and a source at src (V
 * depends on src's 16-byte alignment), into order[0..2]. */
int pe_reduce_order(const pe_reduce_desc* d, const void* src, int64_t* order);

/* Plan executor: the body of every per-shape run_einsum_exec.  Every
 * workspace region a plan uses is written before it is read, so a workspace
 * needs no clearing between calls (or plans). */
int pe_einsum_exec(const pe_einsum_plan* p, const void* in0, const void* in1, float* out,
                   void* ws, void* stream);
/* Workspace bytes a plan needs (>= 256): what pe_einsum_setup allocates, for
 * callers that provide the workspace themselves (no counterpart in the
 * reference, whose setup always allocates). */
int64_t pe_einsum_workspace_bytes(const pe_einsum_plan* p);
/* Allocates the plan's workspace (>= 256 bytes, never NULL on success). */
void* pe_einsum_setup(const pe_einsum_plan* p, void* stream);
/* Waits for the device, then frees a workspace from pe_einsum_setup. */
int pe_einsum_teardown(void* ws);
/* Synchronous one-shot: setup, exec, stream sync, teardown. */
int pe_einsum_run(const pe_einsum_plan* p, const void* in0, const void* in1, float* out,
                  void* stream);

/* Allocation-free plan executor.  No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same kernels and results as
 * pe_einsum_exec, but the workspace is a static device array of
 * PE_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds until the
 * process ends; no hipMalloc, hipFree or allocating library call is made.
 * A plan whose workspace exceeds the limit returns PE_ERR_WORKSPACE (message
 * in pe_last_error) without launching.  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (different streams, or
 * different host threads without ordering) race. */
#define PE_NOALLOC_SCRATCH_BYTES (64ll << 20)
int pe_einsum_exec_noalloc(const pe_einsum_plan* p, const void* in0, const void* in1, float* out,
                           void* stream);

const char* pe_last_error(void);        /* message for the calling thread's last failure */
int pe_device_cu_count(void);           /* compute units of the current device */
const char* pe_version(void);

/* Attainable-peak probe for the measurement harness (no counterpart in the
 * reference): MFMA throughput with no memory traffic, v_mfma_f32_32x32x16_f16
 * (dtype PE_F16) or v_mfma_f32_32x32x2_f32 (PE_F32), on random (random != 0)
 * or constant operands; the clock, and so the rate, depends on the operands'
 * bit activity.  out receives one float per lane (pe_probe_out_len()
 * floats); pe_probe_mfma_flops gives the flops one call performs. */
int pe_probe_mfma(int dtype, int random, int64_t iters, float* out, int64_t out_len, void* stream);
int64_t pe_probe_mfma_flops(int dtype, int64_t iters);
int64_t pe_probe_out_len(void);
/* Launch-floor probe (no counterpart in the reference): enqueues one wave that
 * stores out[0] = 0, the least work a launch can carry; its time per launch
 * in a graph replay is the fixed cost any kernel pays on the device. */
int pe_probe_launch(float* out, void* stream);

/* ---- per-shape entry points (one JIT library per equation/shapes/dtype) ----
 * Declared here with T = void; the generated source defines them with the
 * element type of its dtype. */
#ifndef PE_NO_PER_SHAPE_DECLS
/* reference: templates.py:178-180 -> pto_einsum.h:283-290 (one-shot) */
int run_einsum(const void* input0, const void* input1, float* output, void* stream);
/* reference: templates.py:181-183 -> pto_einsum.h:207-248 */
void* run_einsum_setup(void* stream);
/* reference: templates.py:184-186 -> pto_einsum.h:253-275 */
int run_einsum_exec(const void* input0, const void* input1, float* output, void* workspace,
                    void* stream);
/* reference: templates.py:187-189 -> pto_einsum.h:277-279 */
void run_einsum_teardown(void* workspace);
/* reference: templates.py:166-171 -> pto_einsum_transpose.h:662-678 */
int run_transpose_inp0(const void* input, void* output, void* stream);
int run_transpose_inp1(const void* input, void* output, void* stream);
/* reference: templates.py:172-174 */
int run_transpose_out(const float* input, float* output, void* stream);
/* reference: templates.py:175-177 -> pto_einsum_matmul.h:973-1027 */
int run_batched_matmul(const void* ws0, const void* ws1, float* ws_res, void* stream);
#endif

#ifdef __cplusplus
}
#endif

#endif /* PTO_EINSUM_HIP_H */
