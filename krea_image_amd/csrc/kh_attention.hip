// Flash attention forward for MI355X (gfx950), head dim 128, fp16 / bf16 in and out, fp32 scores, softmax
// and accumulation: the joint image + text attention of the Krea 2 DiT.
//
// Semantics: engine/kernels/attention.metal:131-351 (attention_d128) as dispatched by
// engine/src/metal.mm:193-202 (Metal::attention):
//   O[q, h] = softmax_k(Q[q, h] . K[k, h / group] / sqrt(128) (+ QB[q, h] KB[k, h / group])) V[k, h / group]
//             (* sigmoid(G[q, h]) when a gate is given), optional causal mask key <= q + q_pos0.
// P is rounded to the 16-bit type before P V (attention.metal:272-276). The row sums here add the same
// rounded P (one v_dot2 per key pair) where the reference adds the unrounded p: numerator and denominator
// then see identical weights; the difference is below half a 16-bit ulp per term, unbiased.
//
// Design (CDNA4, v_mfma_f32_32x32x16):
//  * Transposed products: S^T = K Q^T (K is the A operand straight from LDS, Q^T the B operand held in
//    registers for the whole key loop) and O^T += V^T P^T. In the 32 x 32 accumulator layout a lane owns
//    one query column, so the running max / sum and the O rescale are per-lane scalars: no row shuffles
//    except one lane-pair exchange (lane l, l ^ 32) per key block.
//  * P^T is fed to the second MFMA straight from the S^T registers: within a 16-key step the lane's keys are
//    {4h .. 4h+3, 8+4h .. 8+4h+3} (h = lane / 32), and the V^T operand is read in that same key order, so
//    the contraction needs no data movement (the key order inside a step is irrelevant to the sum).
//  * K tiles stream global -> LDS directly (16-byte DMA per lane), rows of 256 B with the 16-byte chunk
//    XOR-swizzled by (row & 15). V tiles are transposed on the way in (4 keys x 8 dims per thread,
//    v_perm_b32 into 8 dims x 4 keys) into V^T rows of 128 B (key order and swizzle: vt_off).
//  * 8 waves x 32 queries per workgroup (one per CU; 4 waves and two per CU with the rank-1 term), 64-key
//    blocks; K tiles double-buffered, V^T tiles triple-buffered (80 KB). Waves 0..3 transpose V. Software pipeline: block b issues S(b), then P V of block b - 1, and
//    the softmax of block b runs on the VALU while those MFMAs execute.
//  * Lazy online softmax (the reference's LAZY_TH idea, attention.metal:33-37): the running max only moves
//    when a block's max exceeds it by more than 8 (log2 units), so most blocks skip the O rescale.
#include <cstdlib>
#include <type_traits>

#include "kh_common.h"
#include "kh_internal.h"

namespace kh {

namespace {

constexpr int D = 128, BKEYS = 64;
constexpr int KT_BYTES = BKEYS * D * 2;   // K tile: 64 rows x 256 B
constexpr int VT_BYTES = D * BKEYS * 2;   // V^T tile: 128 rows x 128 B
constexpr int K_STAGES = 2, V_STAGES = 3;  // V^T lives one block longer: P V of block b - 1 runs in block b
constexpr int LDS_BYTES = K_STAGES * KT_BYTES + V_STAGES * VT_BYTES;  // 80 KB: two workgroups per CU
constexpr float LAZY_TH = 8.0f;
constexpr float M_INIT = -1.0e30f;        // finite: a fully masked block leaves exp2(-inf - M_INIT) = 0

struct AttnArgs {
  const void *Q, *K, *V;
  void* O;
  const void* G;
  const float *QB, *KB;
  int Lq, Lk, heads, ldq, ldk, ldv, ldo, group, q_pos0, ldg, ldqb, ldkb;
  float scale_log2;
};

template <int DT>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (DT == KH_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

// Combine the value of lane l with that of lane l ^ 32 (the two lanes holding the two key halves of one query)
// with v_permlane32_swap: a VALU lane exchange instead of an LDS-routed shuffle on the softmax's critical
// path. Swapping the upper half of one copy of x with the lower half of another leaves x_lo[l % 32] in the
// first and x_hi[l % 32] in the second at every lane, so both lanes compute the same expression. (Written
// as asm: the compiler builtin with one value for both operands folded the two results into one.)
__device__ __forceinline__ void swap_halves(float x, float& lo, float& hi) {
  lo = x;
  hi = x;
  // the wait states around it are the ones the compiler inserts for the builtin form (VALU write -> swap
  // read, swap write -> VALU read); inside asm it cannot see the hazard
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(lo), "+v"(hi));
}
__device__ __forceinline__ float max_halves(float x) {
  float lo, hi;
  swap_halves(x, lo, hi);
  return fmaxf(lo, hi);
}
// max_halves with the max inside the asm: on the asm's outputs fmaxf first canonicalises each operand (two
// extra VALU); v_max_f32 of the two halves is the same value for every non-NaN input
__device__ __forceinline__ float max_halves_fused(float x) {
  float lo = x, hi = x, r;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %1, %2\n\ts_nop 1\n\tv_max_f32 %0, %1, %2"
               : "=v"(r), "+v"(lo), "+v"(hi));
  return r;
}
__device__ __forceinline__ float sum_halves(float x) {
  float lo, hi;
  swap_halves(x, lo, hi);
  return lo + hi;
}

// acc + lo + hi of a packed 16-bit pair (v_dot2c_f32_{f16,bf16} against (1, 1))
template <int DT>
__device__ __forceinline__ float dot2_ones(uint32_t pr, float acc) {
  if constexpr (DT == KH_BF16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, pr), (bf2){(__bf16)1.0f, (__bf16)1.0f}, acc, false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pr), (f16x2){(_Float16)1.0f, (_Float16)1.0f}, acc, false);
  }
}

// V^T row d is 128 B = 8 chunks of 16 B = 16 quads of 4 keys. Key quad kq goes to chunk
// 2 (kq >> 2) + (kq & 1), half (kq >> 1) & 1, so the two quads one MFMA lane needs in key step j
// (4 j + hh and 4 j + 2 + hh) are one 16-byte chunk, 2 j + hh: one ds_read_b128 per operand, already in
// operand order. Chunks are XOR-swizzled by ((d >> 1) ^ (d >> 4)) & 7. LDS serves 16 lanes per cycle for
// 16-byte reads and 32 for 8-byte writes (64 banks x 4 B); with the store order of store_vt, both the
// operand reads (16 consecutive rows, one logical chunk) and the transpose writes hit 64 distinct banks.
__device__ __forceinline__ int vt_off(int d, int kq) {
  return d * 128 + (((2 * (kq >> 2) + (kq & 1)) ^ (((d >> 1) ^ (d >> 4)) & 7)) * 16) + ((kq >> 1) & 1) * 8;
}

// NW waves x 32 queries per workgroup: 4 (two workgroups per CU) or 8 (one per CU; each K / V tile staged in
// LDS then feeds twice the MFMA work).
// AA: the scalar-address form. Wave-uniform values (wave index, LDS stage offsets, K / V block bases) are read
// into scalars; K / V loads of a full block are a scalar base plus per-lane 32-bit offsets computed once (only
// a block reaching past Lk clamps its rows); the V^T transpose writes and operand reads take four per-lane
// offsets each, computed once; the block max of the two lane halves runs inside the lane-swap asm. The same
// values land in the same places: results are bitwise those of the default form. Needs ldk, ldv <= 2^24.
template <int DT, bool GATE, bool BIG, bool CAUSAL, int NW, bool AA = false>
__global__ __launch_bounds__(64 * NW, 8 / NW) void attn_kernel(AttnArgs p) {
  constexpr int BQ = 32 * NW;
  // [K stage 0 | K stage 1 | V^T stage 0 | 1 | 2]
  __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES];
  typedef __attribute__((address_space(3))) void lds_void;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = AA ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  // Workgroup -> (head, query block). The dispatcher deals workgroups round-robin to the 8 XCDs (each
  // with its own L2); ids are remapped so that each XCD walks whole heads in order: its resident
  // workgroups then share one or two heads' K / V (2.4 MB per head at 4608 keys) in their L2.
  const int nqb = (p.Lq + BQ - 1) / BQ, total = nqb * p.heads;
  int wg = blockIdx.x;
  if (total % 8 == 0) wg = (wg % 8) * (total / 8) + wg / 8;
  const int h = wg / nqb, kvh = h / p.group;
  const int qblk = (wg % nqb) * BQ;
  const int q = qblk + wave * 32 + l32;       // this lane's query
  const int qc = min(q, p.Lq - 1);            // clamped (rows >= Lq are computed, never stored)

  // ---- Q^T fragments (B operand): d-step s covers d [16 s, 16 s + 16); lane half hh holds 8 of them ----
  u32x4 qf[8];
  {
    const uint16_t* qp = (const uint16_t*)p.Q + (size_t)qc * p.ldq + h * D + hh * 8;
#pragma unroll
    for (int s = 0; s < 8; s++) qf[s] = *(const u32x4*)(qp + s * 16);
  }
  // rank-1 fp32 term qb[q] kb[k] (BIG): the initial accumulator of each 32-key S^T block is the outer
  // product kb qb^T, one v_mfma_f32_32x32x2_f32 with A = kb (key rows, k-slice 0; the lanes of k-slice 1
  // hold 0) and B = qb (query columns, likewise): it lands in the S^T accumulator layout, needs no LDS and
  // keeps the workgroup at 80 KB (two per CU). The product is exact before the 16-bit products are added.
  const float qb_op = (BIG && hh == 0) ? p.QB[(size_t)qc * p.ldqb + h] : 0.f;

  // key range of this workgroup (causal: up to its last query's visible key)
  int kend = p.Lk;
  if (CAUSAL) kend = max(0, min(p.Lk, qblk + BQ + p.q_pos0));
  const int nblk = (kend + BKEYS - 1) / BKEYS;

  // ---- K tile DMA: instruction r of wave w fills 1 KB = rows 4 (4 r + w) .. +3; lane -> row lane / 16,
  //      chunk slot lane & 15 receives logical chunk (lane & 15) ^ (row & 15) ----
  const uint16_t* kbase = (const uint16_t*)p.K + kvh * D;
  // AA: per-lane 32-bit byte offsets of the K rows within a block (64 rows x ldk x 2 B < 2^31)
  uint32_t koff[16 / NW];
  if constexpr (AA) {
#pragma unroll
    for (int r = 0; r < 16 / NW; r++) {
      const int row = 4 * (NW * r + wave) + (lane >> 4);
      koff[r] = (uint32_t)(row * p.ldk + ((lane & 15) ^ (row & 15)) * 8) * 2u;
    }
  }
  auto issue_k = [&](int b, int buf) {
    if constexpr (AA) {
      const char* kblk = (const char*)kbase + (size_t)b * BKEYS * p.ldk * 2;
      if (b * BKEYS + BKEYS <= p.Lk) {
#pragma unroll
        for (int r = 0; r < 16 / NW; r++)
          __builtin_amdgcn_global_load_lds((const void*)(kblk + koff[r]),
                                           (lds_void*)(lds + buf * KT_BYTES + (NW * r + wave) * 1024), 16, 0, 0);
      } else {
#pragma unroll
        for (int r = 0; r < 16 / NW; r++) {
          const int row = 4 * (NW * r + wave) + (lane >> 4);
          const int krel = min(row, p.Lk - 1 - b * BKEYS);
          const int c = (lane & 15) ^ (row & 15);
          __builtin_amdgcn_global_load_lds((const void*)(kblk + (size_t)(krel * p.ldk + c * 8) * 2),
                                           (lds_void*)(lds + buf * KT_BYTES + (NW * r + wave) * 1024), 16, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16 / NW; r++) {
        const int row = 4 * (NW * r + wave) + (lane >> 4);
        const int key = min(b * BKEYS + row, p.Lk - 1);
        const int c = (lane & 15) ^ (row & 15);
        __builtin_amdgcn_global_load_lds((const void*)(kbase + (size_t)key * p.ldk + c * 8),
                                         (lds_void*)(lds + buf * KT_BYTES + (NW * r + wave) * 1024), 16, 0, 0);
      }
    }
  };
  // ---- V tile: thread -> keys 4 vkq .. 4 vkq + 3, dims 8 vc .. 8 vc + 7. Within a wave the four 16-lane
  //      groups take key quads 4w + {0, 2, 1, 3}, so each half wave writes quads of both 8-byte halves of
  //      a chunk (see vt_off) ----
  const int vlane = tid & 63;
  const int vkq = 4 * (wave & 3) + (((vlane >> 4) & 1) << 1 | ((vlane >> 5) & 1)), vc = vlane & 15;
  const uint16_t* vbase = (const uint16_t*)p.V + kvh * D + vc * 8;
  const uint32_t voff0 = (uint32_t)(4 * vkq * p.ldv) * 2u;  // AA: this lane's first V row in a block (bytes)
  u32x4 vr[4];
  auto load_v = [&](int b) {
    if constexpr (AA) {
      const char* vblk = (const char*)vbase + (size_t)b * BKEYS * p.ldv * 2;
      if (b * BKEYS + BKEYS <= p.Lk) {
#pragma unroll
        for (int r = 0; r < 4; r++) vr[r] = *(const u32x4*)(vblk + (size_t)r * p.ldv * 2 + voff0);
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int krel = min(4 * vkq + r, p.Lk - 1 - b * BKEYS);
          vr[r] = *(const u32x4*)(vblk + (size_t)krel * p.ldv * 2);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int key = min(b * BKEYS + 4 * vkq + r, p.Lk - 1);
        vr[r] = *(const u32x4*)(vbase + (size_t)key * p.ldv);
      }
    }
  };
  // 8 dims x 4 keys: V^T[d][4 vkq .. 4 vkq + 3] as one 8-byte write per d. Write i covers dim
  // 8 vc + (i ^ (vc & 1)): odd-vc lanes swap the two dims of each dword, which only changes the v_perm
  // selector, and spreads the half wave's writes over both row parities.
  const uint32_t sel_lo = (vc & 1) ? 0x07060302u : 0x05040100u, sel_hi = (vc & 1) ? 0x05040100u : 0x07060302u;
  // AA: write i goes to vt_off(8 vc + (i ^ q), vkq), q = vc & 1. The row swizzle of dims 8 vc + j is
  // sw1 ^ (j >> 1) with sw1 = 4 q ^ ((vc >> 1) & 7), so that offset is vst[i >> 1] for even i and
  // vst[i >> 1] + 128 - 256 q for odd i: four per-lane values, computed once.
  uint32_t vst[4];
  const int vdelta = 128 - 256 * (vc & 1);
  if constexpr (AA) {
    const int X = (2 * (vkq >> 2) + (vkq & 1)) ^ (4 * (vc & 1)) ^ ((vc >> 1) & 7);
#pragma unroll
    for (int t = 0; t < 4; t++)
      vst[t] = 1024 * vc + ((vkq >> 1) & 1) * 8 + 256 * t + 16 * (X ^ t) + 128 * (vc & 1);
  }
  auto store_vt = [&](int buf) {
    char* vt = lds + (AA ? __builtin_amdgcn_readfirstlane(K_STAGES * KT_BYTES + buf * VT_BYTES)
                         : K_STAGES * KT_BYTES + buf * VT_BYTES);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int d = vc * 8 + (i ^ (vc & 1));
      const int w = i >> 1;  // dword of the 16-byte row chunk holding dims 2w, 2w + 1
      const uint32_t sel = (i & 1) ? sel_hi : sel_lo;
      const uint32_t lo = __builtin_amdgcn_perm(vr[1][w], vr[0][w], sel);  // keys 4vkq, 4vkq+1 of dim d
      const uint32_t hi = __builtin_amdgcn_perm(vr[3][w], vr[2][w], sel);  // keys 4vkq+2, 4vkq+3
      const uint32_t off = AA ? vst[i >> 1] + ((i & 1) ? vdelta : 0) : (uint32_t)vt_off(d, vkq);
      *(u32x2*)(vt + off) = (u32x2){lo, hi};
    }
  };
  // kb of keys 32 kh + l32 of block b (lanes of k-slice 1 hold 0), loaded one block ahead
  float kbv[2] = {0.f, 0.f};
  auto load_kb = [&](int b) {
    if (BIG && hh == 0) {
#pragma unroll
      for (int kh = 0; kh < 2; kh++) kbv[kh] = p.KB[(size_t)min(b * BKEYS + kh * 32 + l32, p.Lk - 1) * p.ldkb + kvh];
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; db++) o[db] = (f32x16){};
  float m = M_INIT, l = 0.f;

  // O^T += V^T P^T of one block: P^T from registers, V^T from its LDS stage. AA: the operand of (db, j) is
  // vt_off(32 db + l32, 4 j + hh) = 4096 db + voff[j ^ db]: for d = 32 db + l32 the swizzle is sw0 ^ 2 db with
  // sw0 = ((l32 >> 1) ^ (l32 >> 4)) & 7, and XOR by 2 db moves chunk 2 j + hh to 2 (j ^ db) + hh. Four
  // per-lane offsets then serve all 16 reads, with 4096 db as the immediate.
  uint32_t voff[4];
  if constexpr (AA) {
    const int sw0 = ((l32 >> 1) ^ (l32 >> 4)) & 7;
#pragma unroll
    for (int t = 0; t < 4; t++) voff[t] = l32 * 128 + 16 * ((2 * t + hh) ^ sw0);
  }
  auto pv = [&](const u32x4 (&pf)[4], int vbuf) {
    const char* vt = lds + (AA ? __builtin_amdgcn_readfirstlane(K_STAGES * KT_BYTES + vbuf * VT_BYTES)
                               : K_STAGES * KT_BYTES + vbuf * VT_BYTES);
#pragma unroll
    for (int db = 0; db < 4; db++) {
      const int d = db * 32 + l32;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        // operand slots 0..3: key quad 4 j + hh, slots 4..7: quad 4 j + 2 + hh (one chunk, see vt_off)
        const uint32_t off = AA ? voff[j ^ db] + db * 4096 : (uint32_t)vt_off(d, 4 * j + hh);
        const u32x4 vf = *(const u32x4*)(vt + off);
        o[db] = mfma32<DT>(vf, pf[j], o[db]);
      }
    }
  };

  if (nblk > 0) {
    issue_k(0, 0);
    if (wave < 4) load_v(0);
    load_kb(0);
    if (wave < 4) store_vt(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
    lds_barrier();
  }
  // Software pipeline over 64-key blocks: block b issues S(b) = K Q^T, then P V of block b - 1 (its P^T
  // kept in registers, its V^T in the third LDS stage), then the softmax of S(b) runs on the VALU while
  // those MFMAs execute. MASK: the block holds keys >= Lk or (causal) keys above some query's diagonal;
  // only then are scores masked, so full blocks carry no per-score compares or selects.
  u32x4 pf[4];  // P^T of the previous block
  auto process = [&](int b, auto mask_c) {
    constexpr bool MASK = decltype(mask_c)::value;
    const bool has_next = b + 1 < nblk;
    if (has_next) {
      issue_k(b + 1, (b + 1) & 1);
      if (wave < 4) load_v(b + 1);
    }
    const char* kt = lds + (AA ? __builtin_amdgcn_readfirstlane((b & 1) * KT_BYTES) : (b & 1) * KT_BYTES);

    // S^T = K Q^T: st[kh] holds keys 32 kh + 8 (i / 4) + 4 hh + i % 4 (i = 0..15) of query q
    f32x16 st[2];
#pragma unroll
    for (int kh = 0; kh < 2; kh++) {
      st[kh] = BIG ? __builtin_amdgcn_mfma_f32_32x32x2f32(kbv[kh], qb_op, (f32x16){}, 0, 0, 0) : (f32x16){};
      const int krow = kh * 32 + l32;
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const u32x4 kf = *(const u32x4*)(kt + krow * 256 + (((2 * s + hh) ^ (krow & 15)) * 16));
        st[kh] = mfma32<DT>(kf, qf[s], st[kh]);
      }
    }
    if (has_next) load_kb(b + 1);
    if (b > 0) pv(pf, (b - 1) % V_STAGES);

    // block max on the raw scores (the positive scale commutes with max); masked scores are -inf
    float bmax = -INFINITY;
#pragma unroll
    for (int kh = 0; kh < 2; kh++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        float s = st[kh][i];
        if constexpr (MASK) {
          const int key = b * BKEYS + kh * 32 + (i >> 2) * 8 + hh * 4 + (i & 3);
          if (key >= p.Lk || (CAUSAL && key > q + p.q_pos0)) s = -INFINITY;
        }
        st[kh][i] = s;
        bmax = fmaxf(bmax, s);
      }
    bmax = (AA ? max_halves_fused(bmax) : max_halves(bmax)) * p.scale_log2;
    // lazy max update (log2 units): only when some query of the wave grew by more than LAZY_TH (O then
    // already holds block b - 1); the condition is wave-uniform and read into a scalar so the rescale
    // stays a branch
    if (__builtin_amdgcn_readfirstlane(__any(bmax > m + LAZY_TH))) {
      const float m_new = fmaxf(m, bmax);
      asm volatile("" ::: "memory");  // not speculated: the compiler would otherwise multiply by 1 always
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 4; db++) o[db] *= alpha;
    }

    // P^T = exp2(s * scale_log2 - m) as the 16-bit B operand of O^T += V^T P^T (key step j uses
    // st[j / 2][8 (j & 1) ..]); the row sum accumulates the rounded P with v_dot2 (2 keys per op)
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[j >> 1][(j & 1) * 8 + 2 * e], p.scale_log2, -m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[j >> 1][(j & 1) * 8 + 2 * e + 1], p.scale_log2, -m));
        pf[j][e] = pack16<DT>(p0, p1);
        l = dot2_ones<DT>(pf[j][e], l);
      }
    }

    if (has_next) {
      if (wave < 4) store_vt((b + 1) % V_STAGES);  // the stage of block b - 2, whose P V ran in block b - 1
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));  // vmcnt(0): the next K tile has landed
    }
    lds_barrier();
  };
  // blocks [0, nfull) need no mask: all their keys are < Lk and (causal) <= the workgroup's first query
  int nfull = p.Lk / BKEYS;
  if (CAUSAL) nfull = min(nfull, max(0, (qblk + p.q_pos0 + 1) / BKEYS));
  nfull = min(nfull, nblk);
  int b = 0;
  for (; b < nfull; b++) process(b, std::false_type{});
  for (; b < nblk; b++) process(b, std::true_type{});
  if (nblk > 0) pv(pf, (nblk - 1) % V_STAGES);

  // ---- normalise, gate, store: lane holds d = 32 db + 8 g + 4 hh + e of query q ----
  l = sum_halves(l);
  if (q >= p.Lq) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  uint16_t* op = (uint16_t*)p.O + (size_t)q * p.ldo + h * D;
  const uint16_t* gp = GATE ? (const uint16_t*)p.G + (size_t)q * p.ldg + h * D : nullptr;
#pragma unroll
  for (int db = 0; db < 4; db++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int d = db * 32 + g * 8 + hh * 4;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = o[db][g * 4 + e] * inv;
      if (GATE) {
        const u32x2 gv = *(const u32x2*)(gp + d);
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] *= sigmoid_fast(from16<DT>((uint16_t)(gv[e >> 1] >> (16 * (e & 1)))));
      }
      *(u32x2*)(op + d) = (u32x2){pack16<DT>(v[0], v[1]),
                                  pack16<DT>(v[2], v[3])};
    }
}

template <int DT, bool GATE, bool BIG, int NW, bool AA>
hipError_t launch5(bool causal, const AttnArgs& a, hipStream_t st) {
  dim3 grid(((a.Lq + 32 * NW - 1) / (32 * NW)) * a.heads), block(64 * NW);
  if (causal)
    hipLaunchKernelGGL((attn_kernel<DT, GATE, BIG, true, NW, AA>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((attn_kernel<DT, GATE, BIG, false, NW, AA>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int DT, bool GATE, bool BIG, int NW>
hipError_t launch4(bool causal, bool aa, const AttnArgs& a, hipStream_t st) {
  return aa ? launch5<DT, GATE, BIG, NW, true>(causal, a, st) : launch5<DT, GATE, BIG, NW, false>(causal, a, st);
}

template <int DT, bool GATE, bool BIG>
hipError_t launch3(bool causal, bool aa, int nw, const AttnArgs& a, hipStream_t st) {
  return nw == 8 ? launch4<DT, GATE, BIG, 8>(causal, aa, a, st) : launch4<DT, GATE, BIG, 4>(causal, aa, a, st);
}

template <int DT>
hipError_t launch2(bool gate, bool big, bool causal, bool aa, int nw, const AttnArgs& a, hipStream_t st) {
  if (gate)
    return big ? launch3<DT, true, true>(causal, aa, nw, a, st) : launch3<DT, true, false>(causal, aa, nw, a, st);
  return big ? launch3<DT, false, true>(causal, aa, nw, a, st) : launch3<DT, false, false>(causal, aa, nw, a, st);
}

// KH_ATTN_ADDR=1 selects the scalar-address form (attn_kernel AA), bitwise the same results; it needs K / V
// row strides of at most 2^24 elements (per-lane 32-bit offsets within a 64-key block) and the default form
// runs otherwise (read per call)
bool attn_addr(int ldk, int ldv) {
  const char* e = getenv("KH_ATTN_ADDR");
  return e && e[0] == '1' && e[1] == 0 && ldk <= (1 << 24) && ldv <= (1 << 24);
}

// Waves per workgroup: 8 (measured at 4608 tokens: 24 heads 400 -> 324 us; 48 q / 12 kv heads + gate 645 ->
// 616 us; 8704 tokens x 24 heads 1240 -> 1142 us), except with the rank-1 term, where 4 measured faster
// (668 vs 698 us). KH_ATTN_WAVES=4 / 8 overrides (read per call).
int attn_waves(bool big) {
  const char* e = getenv("KH_ATTN_WAVES");
  if (e && (e[0] == '4' || e[0] == '8') && e[1] == 0) return e[0] - '0';
  return big ? 4 : 8;
}

}  // namespace

int attention(hipStream_t st, const void* Q, const void* K, const void* V, void* O, int dtype, int Lq, int Lk,
              int heads, int ldq, int ldk, int ldv, int ldo, int group, int causal, int q_pos0, const void* G,
              int ldg, const float* QB, const float* KB, Err& e) {
  if (dtype != KH_F16 && dtype != KH_BF16) return e.fail("attention: dtype must be f16 or bf16");
  if (Lq <= 0 || Lk <= 0 || heads <= 0) return e.fail("attention: empty shape Lq=%d Lk=%d heads=%d", Lq, Lk, heads);
  if (group <= 0 || heads % group) return e.fail("attention: heads %d not a multiple of group %d", heads, group);
  if (!Q || !K || !V || !O) return e.fail("attention: null Q / K / V / O");
  const int kv_heads = heads / group;
  if (ldq < heads * D || ldo < heads * D || ldk < kv_heads * D || ldv < kv_heads * D)
    return e.fail("attention: row strides too small for %d heads of 128", heads);
  if (ldq % 8 || ldk % 8 || ldv % 8 || ldo % 4) return e.fail("attention: strides must keep 16-byte rows");
  if (((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V) & 15) return e.fail("attention: Q, K, V must be 16-byte aligned");
  if (((uintptr_t)O & 7)) return e.fail("attention: O must be 8-byte aligned");
  if (G && (ldg < heads * D || ldg % 4 || ((uintptr_t)G & 7))) return e.fail("attention: bad gate stride / alignment");
  if ((QB == nullptr) != (KB == nullptr)) return e.fail("attention: QB and KB go together");
  if (Lq > (1 << 24) / 1 || (size_t)Lk * ldk > ((size_t)1 << 31)) return e.fail("attention: too large");
  AttnArgs a{Q, K, V, O, G, QB, KB, Lq, Lk, heads, ldq, ldk, ldv, ldo, group, q_pos0, ldg, heads, kv_heads,
             (float)(1.4426950408889634 / 11.313708498984761)};
  const int nw = attn_waves(QB != nullptr);
  const bool aa = attn_addr(ldk, ldv);
  const hipError_t r = dtype == KH_F16 ? launch2<KH_F16>(G != nullptr, QB != nullptr, causal != 0, aa, nw, a, st)
                                       : launch2<KH_BF16>(G != nullptr, QB != nullptr, causal != 0, aa, nw, a, st);
  if (r != hipSuccess) return e.hip(r, "attention launch");
  return KH_OK;
}

}  // namespace kh
