// step_kernels.hpp -- the non-GEMV kernels of the GPU-resident decode step
// (PrismEngine::step, src/lut/engine_impl.rs:1076-1405, for a Qwen2 graph).
//
// Per token the step runs: k_step_begin; per layer the QKV GEMV (RMS norm
// in its prologue), k_step_attention, the O GEMV (+ residual), the gate/up
// SwiGLU GEMV (RMS norm in its prologue), the down GEMV (+ residual); the
// LM-head GEMV (RMS norm in its prologue).  Everything that changes from
// token to token (token id, position, KV lengths) is read from a StepParams
// block in device memory, which k_step_begin writes, so the launch sequence
// after it is fixed and replays as one HIP graph.
//
// KV cache: the reference's INT8 cache (KVCache, engine_impl.rs:514-584),
// kept in HBM as two planes per layer and matrix: int8 values
// [max_seq][kv_dim] and one fp32 scale per token; a block of the
// reference's byte format is (scale, values).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernels.hpp"

namespace prism {

constexpr int kMaxLayers = 128;

struct StepParams {
  uint32_t token;
  uint32_t pos;
  uint32_t kv_len[kMaxLayers];  // tokens cached per layer before this step
};

// The first kernel of a step (launched with the step's parameters by value,
// ahead of the graph): stores the StepParams block for the graph's kernels
// and writes the embedding row of the step's token into the residual stream:
// lut_embed (compute-core/src/lut/evaluator.rs:176-197; engine_impl.rs:
// 1407-1446): LUT[token][nibble] for the first (D/8)*8 elements, zeros past
// them and for tokens >= vocab.  (As two kernels, the parameters' store and
// the embedding as the graph's first node, every token paid one more
// dependent launch.)
__global__ __launch_bounds__(256) void k_step_begin(StepParams v, StepParams* __restrict__ dst,
                                                    const uint8_t* __restrict__ emb, uint32_t vocab, uint32_t D,
                                                    uint16_t* __restrict__ h) {
  static_assert(sizeof(StepParams) % 4 == 0, "copied as dwords");
  const uint32_t* src = reinterpret_cast<const uint32_t*>(&v);
  for (uint32_t i = threadIdx.x; i < sizeof(StepParams) / 4; i += blockDim.x) reinterpret_cast<uint32_t*>(dst)[i] = src[i];
  const uint32_t tok = v.token;
  const uint32_t keff = (D / 8) * 8;
  for (uint32_t k = threadIdx.x; k < D; k += blockDim.x) {
    uint16_t v = 0;
    if (tok < vocab && k < keff) {
      const uint8_t b = emb[(size_t)vocab * 32 + (size_t)tok * (D / 2) + k / 2];
      const uint32_t nib = (k & 1) ? (b >> 4) : (b & 15u);
      const uint8_t* l = emb + (size_t)tok * 32 + 2 * nib;
      v = (uint16_t)(l[0] | (l[1] << 8));
    }
    h[k] = v;
  }
}

// ---- INT8 KV quantization (KVCache::append's q(), engine_impl.rs:532-556)

// Block-wide max of |x| over n fp16 values held one per thread (threads past
// n pass 0).  `red` holds one float per wave.
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
  for (int w = 1; w < nw; w++) m = fmaxf(m, red[w]);
  return m;
}

// scale = 127 / max|x| (1.0 when max|x| <= 1e-10); q = clamp(round(x * scale)),
// round half away from zero like f32::round.
__device__ __forceinline__ float kv_scale(float max_abs) { return max_abs > 1e-10f ? 127.0f / max_abs : 1.0f; }
__device__ __forceinline__ int8_t kv_q(float x, float scale) {
  float q = roundf(x * scale);
  q = fminf(fmaxf(q, -128.0f), 127.0f);
  return (int8_t)q;
}
// dequant_inline (engine_impl.rs:569-584): f16(q * (1 / s)).
__device__ __forceinline__ float kv_dq(int8_t q, float rs) { return h2f(f2h((float)q * rs)); }

// Quantize `ntok` fp16 rows of kv_dim values into cache slots first, first+1,
// ...: one workgroup per row, kv_dim <= blockDim.x.
__global__ __launch_bounds__(256) void k_kv_quant_rows(const uint16_t* __restrict__ src, uint32_t ntok,
                                                       uint32_t kv_dim, int8_t* __restrict__ q,
                                                       float* __restrict__ scale, uint32_t first) {
  __shared__ float red[4];
  const uint32_t t = blockIdx.x;
  if (t >= ntok) return;
  const uint32_t i = threadIdx.x;
  const float x = i < kv_dim ? h2f(src[(size_t)t * kv_dim + i]) : 0.0f;
  const float s = kv_scale(block_max(fabsf(x), red));
  if (i < kv_dim) q[(size_t)(first + t) * kv_dim + i] = kv_q(x, s);
  if (i == 0) scale[first + t] = s;
}

// ---- attention step

struct AttnArgs {
  const uint16_t* qkv;     // [nh*hd q | kv_dim k | kv_dim v] fp16, this token
  int8_t* kq;              // this layer's K values [max_seq][kv_dim]
  float* ks;               // K scales [max_seq]
  int8_t* vq;
  float* vs;
  const float2* rope;      // (cos, sin) [max_seq][hd/2]
  const StepParams* sp;
  float* part;             // split partials [nh][kAttnSplits][2 + hd] (max, sum, unnormalised out)
  uint32_t layer;
  uint32_t nh, nkv;
};

// kAttnSplits workgroups per query head (flash decoding), kAttnThreads
// threads each, HD = 64.  Follows the engine's step for one layer from the K/V projections
// to the attention output:
//  * RoPE on the head's q only (the engine never rotates K,
//    engine_impl.rs:1211-1218), pair (j, j+32) by the host-built
//    (cos, sin) of pos * 10000^(-2j/64) (evaluator.rs:154-166);
//  * the new token's K and V (whole kv_dim vectors, one scale each) are
//    quantized like KVCache::append by the workgroups whose range holds
//    position kv_len; the one of head 0 writes them to slot kv_len, and each
//    uses its own dequantized copy, so no workgroup waits for another;
//  * attention_cpu (evaluator.rs:104-146) over sl = kv_len + 1 positions:
//    split s of a head takes positions [s*C, (s+1)*C), C = ceil(sl / S).
//    Scores: fp32 dots of fp16 q and dequantized fp16 k (four sequential
//    16-dim folds added pairwise), divided by sqrt(64).
//    A split writes (m, sum_p e^(s_p - m), sum_p e^(s_p - m) v_p) to `part`;
//    the O-projection GEMV's prologue (kEpiAttnIn, attn_combine) rescales
//    the S partials to the head's max, adds them and scales once by
//    1 / (sum + 1e-10); the kernel boundary makes every split's partial
//    visible (device-scope fences inside this kernel would write back and
//    invalidate each XCD's whole L2).  Max is exact; the exp, the
//    sums and the output are fp32 in another order than the reference's folds.
// Latency layout: the loads that gate the setup (q, its RoPE row, the new
// token's K and V, all L2-resident) are issued before the split's K rows and
// V words (HBM), since loads return in issue order.  The new token's max
// |k|, |v| are reductions inside wave 0 (kv_dim <= 256: 4 values per lane).
// One barrier publishes q and the new token's dequantized K/V.  Then each of
// the 16 waves runs an online softmax over its own 16-position slice of
// every pass with wave shuffles only: a score is 4 lanes' sequential folds
// over 16 dims each, added pairwise; lane l owns value dims 4*(l%16)..+3 of
// positions l/16 + 4j, j < 4.  One last barrier combines the waves' (m, sum,
// out) partials into the split's.
// sl <= kAttnSplits * kAttnPassPos * kAttnPasses.
constexpr int kAttnSplits = 4;
constexpr int kAttnThreads = 1024;
constexpr int kAttnPassPos = 256;  // positions per pass: 16 per wave
constexpr int kAttnPasses = 8;
constexpr int kAttnMaxSeq = kAttnSplits * kAttnPassPos * kAttnPasses;

// One DPP step: v's value from the lane that `ctrl` selects; rows outside
// `rows` (and lanes with no source) give `fill`.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f(float v, float fill) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, fill), __builtin_bit_cast(int, v),
                                                               CTRL, ROWS, 0xF, false));
}
// Wave-wide max and sum, the result in every lane: DPP within each row of
// 16 lanes (quad_perm xor 1, xor 2, half-row mirror, row mirror), the row
// broadcasts 15 and 31 into lane 63, and a read of lane 63.  All of it stays
// in the VALU, where a ds_bpermute butterfly costs an LDS round trip per
// step; these reductions sit on the attention's critical path (MI355X,
// config-3 attention graph-launched alone: 5.59 -> 5.19 us per launch).
__device__ __forceinline__ float wave_max(float v) {
  const float ninf = -INFINITY;
  v = fmaxf(v, dpp_f<0xB1, 0xF>(v, ninf));
  v = fmaxf(v, dpp_f<0x4E, 0xF>(v, ninf));
  v = fmaxf(v, dpp_f<0x141, 0xF>(v, ninf));
  v = fmaxf(v, dpp_f<0x140, 0xF>(v, ninf));
  v = fmaxf(v, dpp_f<0x142, 0xA>(v, ninf));
  v = fmaxf(v, dpp_f<0x143, 0xC>(v, ninf));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1, 0xF>(v, 0.0f);
  v += dpp_f<0x4E, 0xF>(v, 0.0f);
  v += dpp_f<0x141, 0xF>(v, 0.0f);
  v += dpp_f<0x140, 0xF>(v, 0.0f);
  v += dpp_f<0x142, 0xA>(v, 0.0f);
  v += dpp_f<0x143, 0xC>(v, 0.0f);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__global__ __launch_bounds__(kAttnThreads) void k_step_attention(AttnArgs a) {
#pragma clang fp contract(off)
  constexpr int HD = 64;
  constexpr int T = kAttnThreads;
  constexpr int NW = T / 64;
  constexpr int S = kAttnSplits;
  constexpr int PW = kAttnPassPos / NW;  // positions per wave per pass (16)
  constexpr int VJ = PW / 4;             // V words per lane per slice
  static_assert(PW == 16, "lane roles assume 16 positions per wave");
  __shared__ float s_q[HD];
  __shared__ float s_knew[HD], s_vnew[HD];
  __shared__ float s_part[NW][2 + HD];

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t h = blockIdx.x / S, sp = blockIdx.x % S;
  const uint32_t kvd = a.nkv * HD;
  const uint32_t kvh = h / (a.nh / a.nkv);
  const uint32_t len0 = a.sp->kv_len[a.layer];
  const uint32_t pos = a.sp->pos;
  const uint32_t sl = len0 + 1;
  const uint32_t C = (sl + S - 1) / S;
  const uint32_t p0 = sp * C;
  const uint32_t p1 = p0 + C < sl ? p0 + C : sl;
  const bool has_new = p0 <= len0 && len0 < p1;  // uniform per workgroup
  const uint32_t last = len0 ? len0 - 1 : 0;    // clamp target for unused loads
  const uint16_t* qh = a.qkv + (size_t)h * HD;
  const uint16_t* knew = a.qkv + (size_t)a.nh * HD;
  const uint16_t* vnew = knew + kvd;
  const uint32_t ps = lane >> 2, qd = lane & 3;     // score roles: position, 16-dim quarter
  const uint32_t dg = lane & 15, psub = lane >> 4;  // value roles

  // ---- setup loads: q and its RoPE row; the new token's K and V
  float qx0 = 0.0f, qx1 = 0.0f;
  float2 cs = make_float2(0.0f, 0.0f);
  if (tid < HD / 2) {
    cs = a.rope[(size_t)pos * (HD / 2) + tid];
    qx0 = h2f(qh[tid]);
    qx1 = h2f(qh[tid + HD / 2]);
  }
  float kn[4], vn[4];
  if (has_new && wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t e = lane + 64 * i;
      kn[i] = e < kvd ? h2f(knew[e]) : 0.0f;
      vn[i] = e < kvd ? h2f(vnew[e]) : 0.0f;
    }
  }
  asm volatile("" ::: "memory");  // the K/V loads below issue after these

  // ---- one pass = kAttnPassPos positions; wave w the slice [base + 16w, +16)
  uint4 kr;
  float krs;
  uint32_t vw[VJ];
  float vrs[VJ];
  auto load_pass = [&](uint32_t base) {
    const uint32_t q0 = base + PW * wave;
    const uint32_t p = q0 + ps;
    const uint32_t pc = p < len0 ? p : last;
    kr = reinterpret_cast<const uint4*>(a.kq + (size_t)pc * kvd + kvh * HD)[qd];
    krs = a.ks[pc];
#pragma unroll
    for (int j = 0; j < VJ; j++) {
      const uint32_t pv = q0 + psub + 4 * j;
      const uint32_t pvc = pv < len0 ? pv : last;
      vw[j] = *reinterpret_cast<const uint32_t*>(a.vq + (size_t)pvc * kvd + kvh * HD + 4 * dg);
      vrs[j] = a.vs[pvc];
    }
  };
  if (p0 < p1) load_pass(p0);

  if (has_new && wave == 0) {
    float kmax = 0.0f, vmax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      kmax = fmaxf(kmax, fabsf(kn[i]));
      vmax = fmaxf(vmax, fabsf(vn[i]));
    }
    const float ksc = kv_scale(wave_max(kmax));
    const float vsc = kv_scale(wave_max(vmax));
    if (h == 0) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t e = lane + 64 * i;
        if (e < kvd) {
          a.kq[(size_t)len0 * kvd + e] = kv_q(kn[i], ksc);
          a.vq[(size_t)len0 * kvd + e] = kv_q(vn[i], vsc);
        }
      }
      if (lane == 0) {
        a.ks[len0] = ksc;
        a.vs[len0] = vsc;
      }
    }
    // this head's 64 dims: element kvh * 64 + lane is value kvh of the lane
    float kh = kn[0], vh = vn[0];
#pragma unroll
    for (int i = 1; i < 4; i++)
      if ((uint32_t)i == kvh) {
        kh = kn[i];
        vh = vn[i];
      }
    s_knew[lane] = kv_dq(kv_q(kh, ksc), 1.0f / ksc);
    s_vnew[lane] = kv_dq(kv_q(vh, vsc), 1.0f / vsc);
  }
  if (tid < HD / 2) {
    s_q[tid] = h2f(f2h(qx0 * cs.x - qx1 * cs.y));
    s_q[tid + HD / 2] = h2f(f2h(qx0 * cs.y + qx1 * cs.x));
  }
  __syncthreads();

  // ---- this wave's online softmax over its slices
  const float den = sqrtf((float)HD);
  float m_run = -INFINITY, s_run = 0.0f;
  float o4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t base = p0; base < p1; base += kAttnPassPos) {
    if (base != p0) load_pass(base);
    const uint32_t q0 = base + PW * wave;
    if (q0 >= p1) continue;  // uniform per wave
    const uint32_t p = q0 + ps;
    float part = 0.0f;
    if (p < len0) {
      const float rs = 1.0f / krs;
      const uint32_t kw[4] = {kr.x, kr.y, kr.z, kr.w};
#pragma unroll
      for (int d = 0; d < 16; d++)
        part += s_q[16 * qd + d] * kv_dq((int8_t)(kw[d / 4] >> (8 * (d % 4))), rs);
    } else {
#pragma unroll
      for (int d = 0; d < 16; d++) part += s_q[16 * qd + d] * s_knew[16 * qd + d];
    }
    // quarters (0+1) + (2+3): the same value in all 4 lanes of a position
    part += dpp_f<0xB1, 0xF>(part, 0.0f);
    part += dpp_f<0x4E, 0xF>(part, 0.0f);
    const float sc = (p < p1) ? part / den : -INFINITY;
    const float m_new = fmaxf(m_run, wave_max(sc));  // finite: the slice holds a position
    const float corr = expf(m_run - m_new);          // 0 on the first slice
    const float e = (p < p1) ? expf(sc - m_new) : 0.0f;
    s_run = s_run * corr + wave_sum(qd == 0 ? e : 0.0f);
    m_run = m_new;
#pragma unroll
    for (int c = 0; c < 4; c++) o4[c] *= corr;
#pragma unroll
    for (int j = 0; j < VJ; j++) {
      const uint32_t pv = q0 + psub + 4 * j;
      const float ev = __shfl(e, (int)(4 * (psub + 4 * j)), 64);
      if (pv >= p1) continue;
      if (pv < len0) {
        const float rs = 1.0f / vrs[j];
#pragma unroll
        for (int c = 0; c < 4; c++) o4[c] += ev * kv_dq((int8_t)(vw[j] >> (8 * c)), rs);
      } else {
#pragma unroll
        for (int c = 0; c < 4; c++) o4[c] += ev * s_vnew[4 * dg + c];
      }
    }
  }

  // ---- waves' partials -> this split's (m, sum, unnormalised output)
#pragma unroll
  for (int c = 0; c < 4; c++) {
    o4[c] += __shfl_xor(o4[c], 16, 64);
    o4[c] += __shfl_xor(o4[c], 32, 64);
  }
  if (psub == 0) {
#pragma unroll
    for (int c = 0; c < 4; c++) s_part[wave][2 + 4 * dg + c] = o4[c];
  }
  if (lane == 0) {
    s_part[wave][0] = m_run;
    s_part[wave][1] = s_run;
  }
  __syncthreads();
  if (tid < HD) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; w++) M = fmaxf(M, s_part[w][0]);
    float tot = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float mw = s_part[w][0];
      const float f = (mw == -INFINITY) ? 0.0f : expf(mw - M);
      tot += s_part[w][1] * f;
      o += s_part[w][2 + tid] * f;
    }
    float* mypart = a.part + ((size_t)h * S + sp) * (2 + HD);
    mypart[2 + tid] = o;
    if (tid == 0) {
      mypart[0] = M;
      mypart[1] = tot;
    }
  }
}

// Attention output element (head h, dim d) from the head's S split partials
// [S][2 + 64]: rescale to the head's max, add, scale once by 1/(sum + 1e-10).
__device__ __forceinline__ float attn_combine(const float* hp, uint32_t d) {
#pragma clang fp contract(off)
  constexpr int S = kAttnSplits;
  float mi[S];
#pragma unroll
  for (int i = 0; i < S; i++) mi[i] = hp[i * 66];
  float M = -INFINITY;
#pragma unroll
  for (int i = 0; i < S; i++) M = fmaxf(M, mi[i]);
  float tot = 0.0f, o = 0.0f;
#pragma unroll
  for (int i = 0; i < S; i++) {
    const float f = (mi[i] == -INFINITY) ? 0.0f : expf(mi[i] - M);
    tot += hp[i * 66 + 1] * f;
    o += hp[i * 66 + 2 + d] * f;
  }
  return o * (1.0f / (tot + 1e-10f));
}

}  // namespace prism
