// Fused linear-attention chain on CDNA4 matrix cores (gfx950):
//
//   out[t,p] = sum_s ((sum_n q[t,n] * k[s,n]) * m[t,s]) * v[s,p]
//
// The reference evaluates this as three einsums with float32 intermediates
// (tests/test_llm_ops.py:81-107, benchmarks/complex/bench_linear_attention.py:62-94):
//   A = einsum("tn,sn->ts", q, k); A = einsum("ts,ts->ts", A, m);
//   out = einsum("ts,sp->tp", A, v)
// which writes and re-reads two T x S float32 intermediates.  Here one launch
// keeps each 32x32 block of A in registers:
//
//   1. S^T block = K_blk . Q_blk^T on MFMA (v_mfma_f32_32x32x16_f16 for float16
//      q/k, v_mfma_f32_32x32x2_f32 for float32), float32 accumulation (float32:
//      in two chains, even / odd k steps, added at the end).  With K as the A operand,
//      lane l ends up holding row t = l%32 of the block and the 16 values
//      s = 8*(r/4) + 4*(l/32) + r%4, r = 0..15.
//   2. Those 16 values are multiplied by the mask in registers (one float32
//      rounding, as the Hadamard step).
//   3. P.V, by default on bfloat16 matrix cores at float32 accuracy: the 16
//      values are split into three bfloat16 terms P0 + P1 + P2 (round to
//      nearest even, each term taking 8 more significant bits, remainders
//      exact; what is left is below 2^-24 |P|) and become the A operands of
//      v_mfma_f32_32x32x16_bf16 k-steps whose k order is permuted to match
//      (step q2, lane half h, slot j <-> s = 16*q2 + 8*(j/4) + 4*h + j%4).
//      V is split the same way when it is staged (two terms, exact, for a
//      float16 V; three for a float32 one), transposed and in that permuted
//      order, so one 16-byte LDS read gives a lane its eight k slots.
//      P.V = sum of Pi.Vj over i + j <= 2: five MFMAs (float16 V) or six,
//      products exact, sums float32; everything left out is below
//      2^-22 |P||V| per product -- the bfloat16x3 technique of emulating
//      float32 products on 16-bit matrix cores.  With `precise` the 16 values
//      instead feed sixteen float32 MFMAs (v_mfma_f32_32x32x2_f32), MFMA j
//      pairing lane half h with s = 8*(j/4) + 4*h + j%4, from a float32
//      transposed V tile.
//
// Blocks of 32 t x 32 s whose mask is zero everywhere are skipped when the q,
// k and v values they would read are finite: their contribution is then
// exactly +-0 (with an inf or a NaN among them the block is computed, so the
// result carries the NaN the chain of einsums would).  The s axis is split over
// blocks for parallelism; partial outputs are summed in split order by the
// GEMM's deterministic reduction, so results are run-to-run identical.
//
// Loads are branch-free (clamped in-bounds address, then a select of zero):
// a load on one side of a data-dependent branch makes the compiler wait for
// it where the branches join, which serialises the prefetch.  For that the
// kernel takes q / k rows as whole 16-byte vectors and mask rows as whole
// 4-element vectors; operands whose rows are not laid out that way (base or
// stride misaligned, N or S not a multiple of the vector) are first copied
// into a zero-padded workspace by pad_rows_kernel.
#include "pe_gemm_kernel.h"

#include <algorithm>
#include <type_traits>

namespace pe {
namespace {

// t rows per block: 32 per wave, four or eight waves (PE_LINATTN_WAVES).
// Eight waves share each staged K / V tile among 256 t rows, which halves
// the K / V traffic through L2 against four.
#ifndef PE_LINATTN_WAVES
#define PE_LINATTN_WAVES 8
#endif
constexpr int kWaves = PE_LINATTN_WAVES;
static_assert(kWaves == 4 || kWaves == 8, "four or eight waves per block");
constexpr int kThreadsLA = 64 * kWaves;
constexpr int kTB = 32 * kWaves;
constexpr int kPB = 128;       // p columns per block (four 32-column MFMA blocks)
constexpr int kSB = 32;        // s per step
constexpr int kVLD = kSB + 4;  // LDS pitch of the transposed float32 V tile (conflict-free 16-byte reads)
constexpr int kVBLD = kSB + 8; // LDS pitch (bf16) of the split V tile: 80-byte rows, conflict-free 16-byte reads

// V tile of one s step, transposed ([p][s]).  Float32 P.V: the float32
// values.  Split P.V: V = t[0] + t[1] (+ t[2]) as NV bfloat16 arrays (two
// terms hold a float16 value exactly, three a float32 one to 2^-24) whose s
// order is permuted so that one 16-byte read gives a lane its eight k slots
// of a 32x32x16 MFMA (see the P.V step).
struct VTileF32 {
    float v[kPB][kVLD];
};
template <int NV>
struct VTileSplit {
    uint16_t t[NV][kPB][kVBLD];
};

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Round-to-nearest-even split of two float32 into NT bfloat16 terms:
// x = t[0] + ... + t[NT-1] + e.  Each term is the bfloat16 nearest to what
// the previous ones left (an 8-bit significand: |remainder| <= 2^-8 |what was
// split|), and every remainder is exact in float32, so |e| <= 2^-(8 NT) |x|:
// 2^-24 |x| for three terms, as fine as float32 itself.  Terms come back
// packed, x0's in the low half: each pair conversion is one
// v_cvt_pk_bf16_f32.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <int NT>
__device__ __forceinline__ void split_bf16x2(float x0, float x1, uint32_t (&t)[NT]) {
    f32x2_t x = {x0, x1};
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        t[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2_t));
        if (i + 1 < NT) {
            const f32x2_t h = {__builtin_bit_cast(float, t[i] << 16), __builtin_bit_cast(float, t[i] & 0xffff0000u)};
            x = x - h;
        }
    }
}

struct LinAttnArgs {
    const void* q;
    const void* k;
    const void* v;
    const void* m;
    float* out;                // final [T][P], or split partials [split][T][P]
    int32_t T, S, P;
    int32_t NP;                // readable q / k row length: whole 16-byte vectors, zero past N
    int32_t SP;                // readable mask row length: whole 4-vectors, zero past S
    int64_t q_ts, k_ss, v_ss, m_ts;
    int32_t s_per_split;       // multiple of kSB
};

// Q / K fragment of one MFMA k step: a 16-byte vector (float16) or one float.
template <typename QK>
struct Frag;

template <>
struct Frag<F16> {
    using type = f16x8;
    static constexpr int KSTEP = 16;
    __device__ __forceinline__ static f32x16 mfma(type a, type b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Frag<F32> {
    using type = float;
    static constexpr int KSTEP = 2;
    __device__ __forceinline__ static f32x16 mfma(type a, type b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};

template <typename V>
__device__ __forceinline__ V zero_unless(bool keep, V x) {
    return keep ? x : V{};
}

// Non-finite tests (an infinity or a NaN: all exponent bits set) on raw
// bits.  nf_bits returns a value that is nonzero when some element of x is
// non-finite: float32 elements test their exponent directly; float16 elements
// are tested two per 32-bit word, the exponent of each half plus 1 reaching
// that half's bit 15 exactly when it was all ones.
__device__ __forceinline__ uint32_t nf_word16(uint32_t w) {
    return ((w & 0x7c007c00u) + 0x04000400u) & 0x80008000u;
}
__device__ __forceinline__ uint32_t nf_word32(uint32_t w) {
    return ((w & 0x7f800000u) + 0x00800000u) & 0x80000000u;
}
template <typename V>
__device__ __forceinline__ uint32_t nf_bits(const V& x) {
    static_assert(sizeof(V) % 4 == 0 || sizeof(V) == 2, "whole words or one float16");
    if constexpr (sizeof(V) == 2) {
        return nf_word16(uint32_t(__builtin_bit_cast(uint16_t, x)));
    } else {
        constexpr int NW = sizeof(V) / 4;
        struct Words {
            uint32_t w[NW];
        };
        const Words ws = __builtin_bit_cast(Words, x);
        const bool f16 = sizeof(x) / sizeof(x[0]) == 2 * NW;
        uint32_t r = 0;
#pragma unroll
        for (int i = 0; i < NW; ++i) r |= f16 ? nf_word16(ws.w[i]) : nf_word32(ws.w[i]);
        return r;
    }
}
__device__ __forceinline__ uint32_t nf_bits(const float& x) {
    return nf_word32(__builtin_bit_cast(uint32_t, x));
}

// K tile of one s step in LDS: kSB rows of COLS elements at a padded pitch
// that keeps the fragment reads conflict-free and 16-byte rows aligned.
// Loaded cooperatively in 16-byte chunks.
template <typename QK, int NSTEPS>
struct KTile {
    static constexpr int COLS = NSTEPS * Frag<QK>::KSTEP;
    static constexpr int PITCH = COLS + (QK::kBytes == 2 ? 8 : 4);
    static constexpr int VEC = 16 / QK::kBytes;
    static constexpr int CPR = COLS / VEC;                 // chunks per row
    static constexpr int PER_THREAD = kSB * CPR / kThreadsLA;
    static_assert(kSB * CPR % kThreadsLA == 0, "chunks split evenly over the block");
};

// NSTEPS: MFMA k steps covering N (N <= NSTEPS * KSTEP); VE / ME: element
// types of v and m; PV32: P.V on float32 MFMAs (else on five or six bfloat16
// MFMAs over the three-term split of P and the two- or three-term split of V).
//
// Per s step (32 s), software-pipelined one step ahead: the V tile (32 x 128,
// staged transposed), the K tile and this lane's mask values of step i+1 are
// loaded into registers (raw element type, converted when committed) while
// step i computes from LDS; two LDS stages mean one barrier per step.
template <typename QK, int NSTEPS, typename VE, typename ME, bool PV32>
__global__ __launch_bounds__(kThreadsLA, 8 / kWaves) void linattn_kernel(LinAttnArgs a) {
    using T = typename QK::T;
    using VT = typename VE::T;
    using MT = typename ME::T;
    using F = Frag<QK>;
    using KT = KTile<QK, NSTEPS>;
    using KChunk = typename Pack<KT::VEC, T>::type;
    using MV = typename Pack<4, MT>::type;
    // bfloat16 terms of V: a float16 value splits exactly into two.
    constexpr int NV = VE::kBytes == 2 ? 2 : 3;
    using VTile = std::conditional_t<PV32, VTileF32, VTileSplit<NV>>;
    __shared__ __attribute__((aligned(16))) VTile vt[2];                     // V tile, transposed: [p][s]
    __shared__ __attribute__((aligned(16))) T kt[2][kSB * KT::PITCH];       // K tile: [s][n]
    __shared__ int nf_step[2];  // per stage: s offset of the last step that staged an inf or NaN

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, l32 = lane & 31;
    const int t0 = blockIdx.x * kTB + wave * 32;
    const int p0 = blockIdx.y * kPB;
    const int s_begin = blockIdx.z * a.s_per_split;
    const int s_end = min(a.S, s_begin + a.s_per_split);
    const int noff = QK::kBytes == 2 ? 8 * h : h;  // this lane's n offset inside a k step

    // Q fragments of this lane's row t (B operand), held for the whole block.
    const int trow = min(t0 + l32, a.T - 1);
    const T* qrow = static_cast<const T*>(a.q) + int64_t(trow) * a.q_ts;
    typename F::type qf[NSTEPS];
#pragma unroll
    for (int kk = 0; kk < NSTEPS; ++kk) {
        const int n = kk * F::KSTEP + noff;
        const bool ok = n < a.NP;
        qf[kk] = zero_unless(ok, *reinterpret_cast<const typename F::type*>(qrow + (ok ? n : 0)));
    }
    // A 32x32 block whose mask is zero contributes exactly +-0 only when its q,
    // k and v values are finite (inf * 0 and NaN give NaN in the chain of
    // einsums): such blocks are computed, not skipped.  The wave's q rows are
    // checked once; k and v per step as they are staged.
    uint32_t q_nf = 0;
#pragma unroll
    for (int kk = 0; kk < NSTEPS; ++kk) q_nf |= nf_bits(qf[kk]);
    const bool wave_q_nf = __any(q_nf != 0u);

    f32x16 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;

    // Registers of the step in flight, and this thread's fixed load addresses.
    // This thread's V column and VROWS consecutive s rows of each step.
    constexpr int VROWS = kSB * kPB / kThreadsLA;
    static_assert(VROWS == 8 || VROWS == 16, "V rows per thread");
    const int vp = tid & 127, vs0 = (tid >> 7) * VROWS;
    // Registers of the step in flight.
    struct Pre {
        VT v[VROWS];
        KChunk k[KT::PER_THREAD];
        MV m[4];
    };
    const VT* vrow0 = static_cast<const VT*>(a.v) + int64_t(vs0) * a.v_ss + min(p0 + vp, a.P - 1);
    const T* krow0[KT::PER_THREAD];
    bool kcol_ok[KT::PER_THREAD];
#pragma unroll
    for (int i = 0; i < KT::PER_THREAD; ++i) {
        const int c = tid + kThreadsLA * i, col = (c % KT::CPR) * KT::VEC;
        kcol_ok[i] = col < a.NP;
        krow0[i] = static_cast<const T*>(a.k) + int64_t(c / KT::CPR) * a.k_ss + (kcol_ok[i] ? col : 0);
    }
    const MT* mrow4 = static_cast<const MT*>(a.m) + int64_t(trow) * a.m_ts + 4 * h;
    const bool k_all_cols = a.NP >= KT::COLS;  // no K chunk lies past N

    // Raw loads only: the zero selects happen when the step is committed, one
    // step later, so nothing waits on the loads here.  A step whose 32 s all
    // lie inside S needs no clamping (the usual case); V columns past P feed
    // only outputs that are never stored, so they are not masked at all.
    auto prefetch = [&](Pre& P, int sb) {
        if (sb + kSB <= a.S) {
            const VT* vp_ = vrow0 + int64_t(sb) * a.v_ss;
#pragma unroll
            for (int i = 0; i < VROWS; ++i) {
                P.v[i] = *vp_;
                vp_ += a.v_ss;
            }
#pragma unroll
            for (int i = 0; i < KT::PER_THREAD; ++i)
                P.k[i] = *reinterpret_cast<const KChunk*>(krow0[i] + int64_t(sb) * a.k_ss);
#pragma unroll
            for (int q = 0; q < 4; ++q) P.m[q] = *reinterpret_cast<const MV*>(mrow4 + sb + 8 * q);
        } else {
#pragma unroll
            for (int i = 0; i < VROWS; ++i)
                P.v[i] = vrow0[int64_t(min(sb + vs0 + i, a.S - 1) - vs0) * a.v_ss];
#pragma unroll
            for (int i = 0; i < KT::PER_THREAD; ++i) {
                const int s = sb + (tid + kThreadsLA * i) / KT::CPR;
                P.k[i] = *reinterpret_cast<const KChunk*>(krow0[i] +
                                                           int64_t(min(s, a.S - 1) - (s - sb)) * a.k_ss);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int s = sb + 8 * q + 4 * h;
                P.m[q] = *reinterpret_cast<const MV*>(mrow4 - 4 * h + (s < a.SP ? s : 0));
            }
        }
    };

    // Writes this thread's VROWS V values (s = vs0 .. vs0+VROWS-1 of column
    // vp) into a stage: float32, or split into bf16 hi / lo at the permuted
    // positions 8*hh + j <-> s = 8*(j/4) + 4*hh + j%4 of each 16-s group.
    auto commit_v = [&](int st, auto val) {
        if constexpr (PV32) {
#pragma unroll
            for (int i = 0; i < VROWS; i += 4) {
                f32x4 w = {val(i), val(i + 1), val(i + 2), val(i + 3)};
                *reinterpret_cast<f32x4*>(&vt[st].v[vp][vs0 + i]) = w;
            }
        } else if constexpr (VROWS == 16) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                uint32_t w[4][NV];
#pragma unroll
                for (int j = 0; j < 8; j += 2)
                    split_bf16x2<NV>(val(8 * (j / 4) + 4 * hh + j % 4), val(8 * ((j + 1) / 4) + 4 * hh + (j + 1) % 4),
                                     w[j / 2]);
#pragma unroll
                for (int e = 0; e < NV; ++e)
                    *reinterpret_cast<u32x4*>(&vt[st].t[e][vp][vs0 + 8 * hh]) = u32x4{w[0][e], w[1][e], w[2][e], w[3][e]};
            }
        } else {
            // Half a 16-s group (a = 0: s 0..7 of the group, a = 1: s 8..15):
            // s = 8a + 4hh + i (i < 4) sits at position 8hh + 4a + i.
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            const int g16 = vs0 & ~15, a8 = (vs0 & 15) >> 3;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                uint32_t w[2][NV];
#pragma unroll
                for (int i = 0; i < 4; i += 2) split_bf16x2<NV>(val(4 * hh + i), val(4 * hh + i + 1), w[i / 2]);
#pragma unroll
                for (int e = 0; e < NV; ++e)
                    *reinterpret_cast<u32x2*>(&vt[st].t[e][vp][g16 + 8 * hh + 4 * a8]) = u32x2{w[0][e], w[1][e]};
            }
        }
    };

    // One step from registers P (loaded one step earlier) into LDS stage
    // `stage`, then its MFMAs; P is refilled with step sb + kSB.
    auto step = [&](Pre& P, const int sb, const int stage) {
        // Commit the prefetched step to this stage (its readers from two steps
        // ago passed the previous barrier after finishing), zeroing what lies
        // past S or N.
        const bool full = sb + kSB <= a.S;
        float mv[16];
        // Non-finite k / v values this thread stages: k words tested on their
        // bits; v values through vz = fma(v, 0, vz), which stays +0 for finite
        // v and becomes NaN after any inf or NaN (one instruction per value).
        uint32_t kv_nf = 0;
        float vz = 0.0f;
        if (full) {
            commit_v(stage, [&](int i) { return float(P.v[i]); });
#pragma unroll
            for (int i = 0; i < VROWS; ++i) vz = __builtin_fmaf(float(P.v[i]), 0.0f, vz);
#pragma unroll
            for (int i = 0; i < KT::PER_THREAD; ++i) {
                const int c = tid + kThreadsLA * i;
                const KChunk kc = k_all_cols ? P.k[i] : zero_unless(kcol_ok[i], P.k[i]);
                kv_nf |= nf_bits(kc);
                *reinterpret_cast<KChunk*>(&kt[stage][(c / KT::CPR) * KT::PITCH + (c % KT::CPR) * KT::VEC]) = kc;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < 4; ++i) mv[4 * q + i] = float(P.m[q][i]);
        } else {
            commit_v(stage, [&](int i) { return sb + vs0 + i < a.S ? float(P.v[i]) : 0.0f; });
#pragma unroll
            for (int i = 0; i < VROWS; ++i) vz = __builtin_fmaf(sb + vs0 + i < a.S ? float(P.v[i]) : 0.0f, 0.0f, vz);
#pragma unroll
            for (int i = 0; i < KT::PER_THREAD; ++i) {
                const int c = tid + kThreadsLA * i;
                const bool ok = sb + c / KT::CPR < a.S && kcol_ok[i];
                const KChunk kc = zero_unless(ok, P.k[i]);
                kv_nf |= nf_bits(kc);
                *reinterpret_cast<KChunk*>(&kt[stage][(c / KT::CPR) * KT::PITCH + (c % KT::CPR) * KT::VEC]) = kc;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const bool ok = sb + 8 * q + 4 * h < a.SP;
#pragma unroll
                for (int i = 0; i < 4; ++i) mv[4 * q + i] = ok ? float(P.m[q][i]) : 0.0f;
            }
        }
        // A wave that stages an inf or NaN marks the step (its s offset) in
        // the stage's flag, read after the barrier (and after the next
        // step's loads are issued) by the waves whose mask block is zero.
        // Marks never need clearing: each step writes its own s offset, and
        // the slot is rewritten two steps later, after every wave read it.
        if (__any(kv_nf != 0u || vz != 0.0f) && lane == 0) nf_step[stage] = sb;
        __syncthreads();
        if (sb + kSB < s_end) prefetch(P, sb + kSB);

        // Any mask value other than +-0 (or of the bits, sign dropped).
        uint32_t mbits = 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) mbits |= __builtin_bit_cast(uint32_t, mv[r]);
        if (__any((mbits << 1) != 0u) || wave_q_nf || nf_step[stage] == sb) {
            // 1. S^T block: rows s (this lane: 16 of them), column t = l32.
            //    float16: one accumulation chain (dependent 32x32 MFMAs issue
            //    back to back); float32 (64 k steps): two, even / odd.
            const T* krow = &kt[stage][l32 * KT::PITCH + noff];
            constexpr int NCH = QK::kBytes == 2 ? 1 : 2;
            f32x16 sacc[NCH];
#pragma unroll
            for (int c = 0; c < NCH; ++c)
#pragma unroll
                for (int r = 0; r < 16; ++r) sacc[c][r] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < NSTEPS; ++kk) {
                const typename F::type kf = *reinterpret_cast<const typename F::type*>(krow + kk * F::KSTEP);
                sacc[kk % NCH] = F::mfma(kf, qf[kk], sacc[kk % NCH]);
            }
            // 2. Mask product (float32, one rounding).
            float av[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) av[r] = (NCH == 1 ? sacc[0][r] : sacc[0][r] + sacc[NCH - 1][r]) * mv[r];
            // 3. out[t, p] += sum_s A[t, s] v[s, p].  The four 32-column blocks
            //    are interleaved: four independent chains.
            if constexpr (PV32) {
                // float32 MFMA j takes s = 8*(j/4) + 4*h + j%4.
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    f32x4 vf[4];
#pragma unroll
                    for (int jb = 0; jb < 4; ++jb)
                        vf[jb] = *reinterpret_cast<const f32x4*>(&vt[stage].v[32 * jb + l32][8 * q + 4 * h]);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int jb = 0; jb < 4; ++jb)
                            acc[jb] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[4 * q + i], vf[jb][i], acc[jb], 0, 0, 0);
                }
            } else {
                // bf16 32x32x16 MFMA step q2 covers s = 16*q2 .. 16*q2+15:
                // lane half h, k slot j holds register r = 8*q2 + j, i.e.
                // s = 16*q2 + 8*(j/4) + 4*h + j%4, matching the V positions.
                // P = P0 + P1 + P2 and V = V0 + V1 (+ V2) in bfloat16 terms;
                // P.V = sum of Pi.Vj over i + j <= 2 (products exact, float32
                // sums).  Left out: the split remainders (<= 2^-24 |P| and
                // |V|) and the terms with i + j > 2 (each <= 2^-24 |P||V|,
                // one for a float16 V, three for a float32 one): at most
                // 2^-22 |P||V| per product, float32's own rounding scale.
#pragma unroll
                for (int q2 = 0; q2 < 2; ++q2) {
                    uint32_t w[4][3];
#pragma unroll
                    for (int j = 0; j < 8; j += 2) split_bf16x2<3>(av[8 * q2 + j], av[8 * q2 + j + 1], w[j / 2]);
                    bf16x8 pt[3];
#pragma unroll
                    for (int e = 0; e < 3; ++e) pt[e] = __builtin_bit_cast(bf16x8, u32x4{w[0][e], w[1][e], w[2][e], w[3][e]});
#pragma unroll
                    for (int jb = 0; jb < 4; ++jb) {
                        bf16x8 vv[NV];
#pragma unroll
                        for (int e = 0; e < NV; ++e)
                            vv[e] = *reinterpret_cast<const bf16x8*>(&vt[stage].t[e][32 * jb + l32][16 * q2 + 8 * h]);
#pragma unroll
                        for (int i = 0; i < 3; ++i)
#pragma unroll
                            for (int j = 0; j < NV; ++j)
                                if (i + j <= 2) acc[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pt[i], vv[j], acc[jb], 0, 0, 0);
                    }
                }
            }
        }
    };

    // (A deeper register prefetch, two steps ahead, measured no faster on
    // config 5 and spilled in the float32-q/k instantiations.)
    if (tid < 2) nf_step[tid] = -1;  // no step yet (s offsets are >= 0)
    __syncthreads();
    Pre pre;
    if (s_begin < s_end) prefetch(pre, s_begin);
    for (int sb = s_begin, stage = 0; sb < s_end; sb += kSB, stage ^= 1) step(pre, sb, stage);

    // Store: lane l, register r holds out[t0 + 8*(r/4) + 4*h + r%4][p0 + 32*jb + l32].
    float* out = a.out + int64_t(blockIdx.z) * a.T * a.P;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        const int p = p0 + 32 * jb + l32;
        if (p >= a.P) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (t < a.T) out[int64_t(t) * a.P + p] = acc[jb][r];
        }
    }
}

// dst[r][c] = c < cols ? src[r * src_stride + c] : 0, for c < pitch.
template <typename W>
__global__ __launch_bounds__(256) void pad_rows_kernel(const W* __restrict__ src, int64_t src_stride, W* __restrict__ dst,
                                                       int64_t rows, int64_t cols, int64_t pitch) {
    const int64_t n = rows * pitch;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
        const int64_t r = i / pitch, c = i - r * pitch;
        dst[i] = c < cols ? src[r * src_stride + c] : W(0);
    }
}

int64_t round_up(int64_t x, int64_t m) { return ceil_div(x, m) * m; }

// Workspace: split partials, then zero-padded copies of the operands whose
// rows the kernel cannot read as whole vectors.
struct Plan {
    int nsplit;
    int s_per_split;
    bool stage_q, stage_k, stage_m;
    int64_t NP, SP;
    int64_t q_off, k_off, m_off;
    int64_t ws_bytes;
};

Plan plan(const pe_linattn_desc& d, const void* q, const void* k, const void* m) {
    Plan p{};
    const int64_t blocks_tp = std::max<int64_t>(1, ceil_div(d.T, kTB) * ceil_div(d.P, kPB));  // (empty outputs: nothing runs)
    const int64_t sblocks = std::max<int64_t>(1, ceil_div(d.S, kSB));
    // About eight waves per CU: two blocks of four or one of eight.
    int64_t split = d.split > 0 ? d.split : ceil_div(int64_t(cu_count()) * (8 / kWaves), blocks_tp);
    split = std::max<int64_t>(1, std::min(split, sblocks));
    p.s_per_split = int(ceil_div(sblocks, split) * kSB);
    p.nsplit = int(ceil_div(std::max<int64_t>(d.S, 1), p.s_per_split));
    const int qb = d.qk_dtype == PE_F16 ? 2 : 4, mb = d.m_dtype == PE_F16 ? 2 : 4;
    const int qvec = 16 / qb;
    p.NP = round_up(d.N, qvec);
    p.SP = round_up(d.S, 4);
    // A null pointer (the size query) is taken as aligned: the workspace size
    // covers operands whose base addresses are 16-byte aligned.
    p.stage_q = (q && !aligned(q, 16)) || d.q_ts % qvec != 0 || d.N % qvec != 0;
    p.stage_k = (k && !aligned(k, 16)) || d.k_ss % qvec != 0 || d.N % qvec != 0;
    p.stage_m = (m && !aligned(m, 4 * mb)) || d.m_ts % 4 != 0 || d.S % 4 != 0;
    int64_t off = p.nsplit > 1 ? round_up(int64_t(p.nsplit) * d.T * d.P * 4, 256) : 0;
    p.q_off = off; if (p.stage_q) off += round_up(d.T * p.NP * qb, 256);
    p.k_off = off; if (p.stage_k) off += round_up(d.S * p.NP * qb, 256);
    p.m_off = off; if (p.stage_m) off += round_up(d.T * p.SP * mb, 256);
    p.ws_bytes = off;
    return p;
}

int validate(const pe_linattn_desc& d) {
    auto dt_ok = [](int x) { return x == PE_F32 || x == PE_F16; };
    if (!dt_ok(d.qk_dtype) || !dt_ok(d.v_dtype) || !dt_ok(d.m_dtype))
        return fail(PE_ERR_UNSUPPORTED, "linear_attention: dtypes must be PE_F32 or PE_F16");
    if (d.T < 0 || d.S < 0 || d.N < 0 || d.P < 0) return fail(PE_ERR_INVALID, "linear_attention: negative extent");
    if (d.split < 0) return fail(PE_ERR_INVALID, "linear_attention: split must be >= 0");
    if (d.precise != 0 && d.precise != 1) return fail(PE_ERR_INVALID, "linear_attention: precise must be 0 or 1");
    if (d.reserved != 0) return fail(PE_ERR_INVALID, "linear_attention: reserved field must be 0");
    const int64_t nmax = d.qk_dtype == PE_F16 ? 256 : 128;
    if (d.N > nmax) return fail(PE_ERR_UNSUPPORTED, "linear_attention: N above " + std::to_string(nmax));
    if (d.T >= (int64_t(1) << 31) || d.S >= (int64_t(1) << 31) || d.P >= (int64_t(1) << 31) ||
        d.T * d.P >= (int64_t(1) << 32))
        return fail(PE_ERR_UNSUPPORTED, "linear_attention: extents too large");
    if (d.q_ts < 0 || d.k_ss < 0 || d.v_ss < 0 || d.m_ts < 0)
        return fail(PE_ERR_INVALID, "linear_attention: negative stride");
    if (d.T == 0 || d.P == 0 || d.S == 0 || d.N == 0) return PE_OK;
    if ((d.T - 1) * d.q_ts + d.N > d.q_numel) return fail(PE_ERR_BOUNDS, "linear_attention: q strides address past its extent");
    if ((d.S - 1) * d.k_ss + d.N > d.k_numel) return fail(PE_ERR_BOUNDS, "linear_attention: k strides address past its extent");
    if ((d.S - 1) * d.v_ss + d.P > d.v_numel) return fail(PE_ERR_BOUNDS, "linear_attention: v strides address past its extent");
    if ((d.T - 1) * d.m_ts + d.S > d.m_numel) return fail(PE_ERR_BOUNDS, "linear_attention: m strides address past its extent");
    return PE_OK;
}

template <typename QK, int NSTEPS, typename VE, typename ME>
hipError_t launch(const LinAttnArgs& a, bool pv32, dim3 grid, hipStream_t s) {
    if (pv32)
        hipLaunchKernelGGL((linattn_kernel<QK, NSTEPS, VE, ME, true>), grid, dim3(kThreadsLA), 0, s, a);
    else
        hipLaunchKernelGGL((linattn_kernel<QK, NSTEPS, VE, ME, false>), grid, dim3(kThreadsLA), 0, s, a);
    return hipGetLastError();
}

template <typename QK, int NSTEPS>
hipError_t launch_vm(const LinAttnArgs& a, int vdt, int mdt, bool pv32, dim3 grid, hipStream_t s) {
    if (vdt == PE_F16)
        return mdt == PE_F16 ? launch<QK, NSTEPS, F16, F16>(a, pv32, grid, s) : launch<QK, NSTEPS, F16, F32>(a, pv32, grid, s);
    return mdt == PE_F16 ? launch<QK, NSTEPS, F32, F16>(a, pv32, grid, s) : launch<QK, NSTEPS, F32, F32>(a, pv32, grid, s);
}

hipError_t pad_rows(const void* src, int64_t stride, void* dst, int64_t rows, int64_t cols, int64_t pitch,
                    int elem_bytes, hipStream_t s) {
    const int grid = int(std::max<int64_t>(1, std::min<int64_t>(ceil_div(rows * pitch, 256), cu_count() * 16)));
    if (elem_bytes == 2)
        hipLaunchKernelGGL(pad_rows_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, static_cast<const uint16_t*>(src),
                           stride, static_cast<uint16_t*>(dst), rows, cols, pitch);
    else
        hipLaunchKernelGGL(pad_rows_kernel<uint32_t>, dim3(grid), dim3(256), 0, s, static_cast<const uint32_t*>(src),
                           stride, static_cast<uint32_t*>(dst), rows, cols, pitch);
    return hipGetLastError();
}

}  // namespace
}  // namespace pe

extern "C" int64_t pe_linear_attention_workspace_bytes(const pe_linattn_desc* d) {
    if (!d || pe::validate(*d) != PE_OK) return 0;
    if (d->T == 0 || d->P == 0 || d->S == 0 || d->N == 0) return 0;  // nothing staged or split
    return pe::plan(*d, nullptr, nullptr, nullptr).ws_bytes;
}

extern "C" int pe_linear_attention(const pe_linattn_desc* d, const void* q, const void* k, const void* v,
                                   const void* m, float* out, void* ws, int64_t ws_bytes, void* stream) {
    using namespace pe;
    if (!d) return fail(PE_ERR_INVALID, "linear_attention: null descriptor");
    int st = validate(*d);
    if (st != PE_OK) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (d->T == 0 || d->P == 0) return PE_OK;

    ReduceArgs r{};
    r.c = out;
    r.per_split = uint32_t(d->T * d->P);
    r.n_div.init(uint32_t(d->P));
    r.m_div.init(uint32_t(d->T));
    r.c_ms = d->P;
    r.c_ns = 1;
    r.nbatch = 0;
    r.store_nt = 0;
    if (d->S == 0 || d->N == 0) {
        // Empty sums: every A[t, s] is +0 (N = 0) or there is no s at all,
        // so every output is +0 (operands are not read).
        r.nsplit = 0;
        r.partial = nullptr;
        PE_CHECK_HIP(launch_splitk_reduce(r, s));
        return PE_OK;
    }
    const Plan pl = plan(*d, q, k, m);
    if (pl.ws_bytes > 0 && (!ws || ws_bytes < pl.ws_bytes))
        return fail(PE_ERR_WORKSPACE, "linear_attention: workspace missing or too small (" +
                                          std::to_string(pl.ws_bytes) + " bytes needed; operands not "
                                          "16-byte aligned need more than the size query reports)");

    LinAttnArgs a{};
    char* wsb = static_cast<char*>(ws);
    const int qb = d->qk_dtype == PE_F16 ? 2 : 4, mb = d->m_dtype == PE_F16 ? 2 : 4;
    a.q = q; a.k = k; a.v = v; a.m = m;
    a.q_ts = d->q_ts; a.k_ss = d->k_ss; a.v_ss = d->v_ss; a.m_ts = d->m_ts;
    if (pl.stage_q) {
        PE_CHECK_HIP(pad_rows(q, d->q_ts, wsb + pl.q_off, d->T, d->N, pl.NP, qb, s));
        a.q = wsb + pl.q_off;
        a.q_ts = pl.NP;
    }
    if (pl.stage_k) {
        PE_CHECK_HIP(pad_rows(k, d->k_ss, wsb + pl.k_off, d->S, d->N, pl.NP, qb, s));
        a.k = wsb + pl.k_off;
        a.k_ss = pl.NP;
    }
    if (pl.stage_m) {
        PE_CHECK_HIP(pad_rows(m, d->m_ts, wsb + pl.m_off, d->T, d->S, pl.SP, mb, s));
        a.m = wsb + pl.m_off;
        a.m_ts = pl.SP;
    }
    a.out = pl.nsplit > 1 ? reinterpret_cast<float*>(wsb) : out;
    a.T = int32_t(d->T); a.S = int32_t(d->S); a.P = int32_t(d->P);
    a.NP = int32_t(pl.NP);
    a.SP = int32_t(pl.SP);
    a.s_per_split = pl.s_per_split;
    const dim3 grid(uint32_t(ceil_div(d->T, kTB)), uint32_t(ceil_div(d->P, kPB)), uint32_t(pl.nsplit));
    hipError_t e;
    const bool pv32 = d->precise != 0;
    if (d->qk_dtype == PE_F16)
        e = d->N <= 128 ? launch_vm<F16, 8>(a, d->v_dtype, d->m_dtype, pv32, grid, s)
                        : launch_vm<F16, 16>(a, d->v_dtype, d->m_dtype, pv32, grid, s);
    else
        e = launch_vm<F32, 64>(a, d->v_dtype, d->m_dtype, pv32, grid, s);
    PE_CHECK_HIP(e);
    if (pl.nsplit > 1) {
        r.nsplit = pl.nsplit;
        r.partial = reinterpret_cast<const float*>(wsb);
        PE_CHECK_HIP(launch_splitk_reduce(r, s));
    }
    return PE_OK;
}
