// Decoding against a key / value cache kept in a class-A basis (gfx950).
//
// The reference relabels tokens for prefill only and leaves decoding open: new keys
// arrive in original order and would have to be inserted at permuted positions
// (docs/NOTES.md:2145-2153, 2201-2203).  With a cache of fixed capacity C, a multiple
// of s, the residue-s basis gives every class its own segment of Q = C / s rows, and
// the token at original position t sits at row (t mod s) Q + t div s: the end of its
// class's segment.  Appending is one row write per token and tensor; cached rows never
// move.  s = 1 is the identity basis.
//
// pa_kv_append writes the new rows.  pa_decode_fwd attends up to 8 query rows at
// original positions qpos0 .. qpos0 + nq - 1 to the first `length` tokens under any
// pa_mask, split over the keys: one work-group per (share of one class's segment, head)
// writes a normalised partial and its log-sum-exp into the workspace, and a second
// kernel merges the partials.  Keys are visited in 64-key blocks, one per wave and
// one key per lane: a block with no live pair is not read at all, and in a block only
// the live keys' K and V rows are read.  The bytes moved follow the live pairs in
// either basis; what the relabelling saves is the visits to blocks with few live keys.
#include <math.h>

#include <mutex>
#include <numeric>

#include "common.hpp"

namespace pa {
namespace {

constexpr int kDecMaxQ = 8;     // query rows per call
constexpr int kDecWaves = 4;    // waves per work-group
constexpr int kDecTarget = 512;    // work-groups a split plan aims for (two per CU, one round)
constexpr int kMergeMax = kDecTarget;  // splits per (head, query) the merge takes
constexpr int kMaxResidue = 4096;       // classes of the largest residue basis a cache may use

typedef uint32_t du4 __attribute__((ext_vector_type(4)));

struct DecK {
  const char* q;
  int64_t q_sb, q_sn;  // elements
  char* k;  // the cache (written only for the rows this call appends)
  char* v;
  int64_t c_sb, c_sn;  // elements
  int64_t qpos0, length, Q, groups;  // groups: group numbers per class (see plan_of)
  int32_t nq, s, n_split;             // n_split: work-groups per head
  float c;  // scale * log2(e)
  Pred pred;
  float* o_part;    // [BH][n_split][nq][D]
  float* lse_part;  // [BH][n_split][nq]
  // tokens appended by this call (n_new = 0: none): their K / V rows are read from
  // k_new / v_new, and the work-group owning a new row writes it to the cache
  const char* k_new;
  const char* v_new;
  int64_t new_sb, new_sn;  // bytes
  int64_t n_new, new_pos0;
};

// 16 bytes of a K row against 16 bytes of a query row, accumulated in fp32; one or two
// output dimensions of a V row as floats.
template <typename T>
struct Dec;
template <>
struct Dec<__bf16> {
  typedef __bf16 h2 __attribute__((ext_vector_type(2)));
  __device__ static float dot16(du4 k, du4 q, float acc) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t kw = k[e], qw = q[e];  // (scalar copies: bit-casting a vector element reads element 0)
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(h2, kw), __builtin_bit_cast(h2, qw), acc, false);
    }
    return acc;
  }
  // the lane's V word: one (low 16 bits) or two elements
  __device__ static float lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
  __device__ static float hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
};
template <>
struct Dec<_Float16> {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  __device__ static float dot16(du4 k, du4 q, float acc) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t kw = k[e], qw = q[e];
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, kw), __builtin_bit_cast(h2, qw), acc, false);
    }
    return acc;
  }
  __device__ static float lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu)); }
  __device__ static float hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }
};
template <>
struct Dec<float> {
  __device__ static float dot16(du4 k, du4 q, float acc) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t kw = k[e], qw = q[e];
      acc = __builtin_fmaf(__builtin_bit_cast(float, kw), __builtin_bit_cast(float, qw), acc);
    }
    return acc;
  }
  __device__ static float lo(uint32_t w) { return __builtin_bit_cast(float, w); }
  __device__ static float hi(uint32_t w) { return __builtin_bit_cast(float, w); }
};

// LDS DMA of 16 bytes per lane: lane l writes LDS[m0 + 16 l] from gbase + voff (one wait
// state between the scalar write of M0 and the DMA that reads it).
__device__ __forceinline__ void lds_dma16(uint32_t m0, const char* gbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(voff), "s"(gbase)
               : "m0");
}

// The same from a 64-bit address per lane.
__device__ __forceinline__ void lds_dma16_va(uint32_t m0, const char* p) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(p) : "m0");
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// One work-group per (split, head).  Wave w takes the blocks b0 = 256 k + 64 w of the
// groups (class, k) the split takes.  LIST: it lists the blocks' live keys, then, 64 listed
// keys at a time, lane l scores key l from its K row; else lane l scores key b0 + l of each
// block that holds a live key.  The keys' V rows go by LDS DMA into the wave's 64-row
// buffer, and for P.V the lanes own output dimensions (D / 64 each).  MQ = 1 is the
// single-query case (fewer registers), MQ = kDecMaxQ takes 2..8 queries.
template <typename T, int D, int MQ, bool LIST>
__global__ __launch_bounds__(256) void decode_kernel(const DecK a) {
  constexpr int ESZ = sizeof(T);
  constexpr int RB = D * ESZ;     // row bytes
  constexpr int NC = RB / 16;     // 16-byte chunks per row
  constexpr int DPL = D / 64;     // output dimensions per lane
  constexpr int LPR = RB / 16;    // DMA lanes per row
  constexpr int RPI = 64 / LPR;   // rows per DMA instruction
  // the waves' V buffers; after the key loop the same LDS holds the cross-wave partials
  __shared__ __attribute__((aligned(16))) char vbuf[kDecWaves * 64 * RB];
  __shared__ __attribute__((aligned(16))) char q_lds[MQ * RB];
  __shared__ float red_m[kDecWaves][MQ];
  __shared__ float red_l[kDecWaves][MQ];
  __shared__ int32_t kl_row[kDecWaves][128];  // each wave's list of live keys
  __shared__ uint32_t kl_lv[kDecWaves][128];
  static_assert(sizeof(float) * kDecWaves * MQ * D <= sizeof(vbuf), "partials fit the V buffers");
  float(*red_o)[MQ][D] = reinterpret_cast<float(*)[MQ][D]>(vbuf);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int split = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int nq = MQ == 1 ? 1 : a.nq;

  for (int u = tid; u < nq * NC; u += 256) {
    const int i = u / NC, cc = u - (u / NC) * NC;
    *reinterpret_cast<du4*>(q_lds + i * RB + 16 * cc) =
        *reinterpret_cast<const du4*>(a.q + (bh * a.q_sb + (int64_t)i * a.q_sn) * ESZ + 16 * cc);
  }
  __syncthreads();

  // this split's keys: the head's segments are cut into groups of 256 entries, numbered
  // g = class * groups + k (entries 256 k .. 256 k + 255 of the class's segment; a number
  // past the segment's end is an empty group), and the split takes the groups split,
  // split + n_split, split + 2 n_split, ..., one 64-key block per wave and group.  A run of
  // live keys (a window at the end of the context, or the one class that holds a lattice
  // row's keys) is thus spread over many work-groups, and so are the groups at one place k
  // of every class (groups and n_split have no common factor).
  const uint32_t n_groups = (uint32_t)(a.s * a.groups);
  const int64_t rowb = a.c_sn * ESZ;
  const char* knew = a.n_new ? a.k_new + bh * a.new_sb : nullptr;
  const char* vnew = a.n_new ? a.v_new + bh * a.new_sb : nullptr;

  // The appended rows this work-group owns (entry e of this class's segment in one of its
  // groups) go to the cache: thread u copies 16-byte unit u % NC of the K (u < NC) or V
  // row.  Nothing in this launch reads them back from the cache: the keys' lanes below
  // take them from k_new / v_new.
  for (int64_t j = 0; j < a.n_new; ++j) {
    const int64_t t = a.new_pos0 + j;
    const int64_t e = t / a.s;
    const int64_t ncls = t - e * a.s;
    if ((ncls * a.groups + (e >> 8)) % a.n_split != split) continue;
    if (tid < 2 * NC) {
      const int uu = tid % NC;
      const char* src = (tid < NC ? knew : vnew) + j * a.new_sn + 16 * uu;
      char* dst = (tid < NC ? a.k : a.v) + (bh * a.c_sb + ncls * a.Q * a.c_sn) * ESZ + e * rowb + 16 * uu;
      *reinterpret_cast<du4*>(dst) = *reinterpret_cast<const du4*>(src);
    }
  }

  float m[MQ], lsum[MQ], o[MQ][DPL];
#pragma unroll
  for (int i = 0; i < MQ; ++i) {
    m[i] = -1e30f;  // finite: exp2(m - m_new) is 0, never NaN
    lsum[i] = 0.f;
#pragma unroll
    for (int d = 0; d < DPL; ++d) o[i][d] = 0.f;
  }

  const char* kh = a.k + bh * a.c_sb * ESZ;
  const char* vh = a.v + bh * a.c_sb * ESZ;
  const uint32_t vbw = (uint32_t)(uintptr_t)(vbuf + w * 64 * RB);
  const char* vbuf_w = vbuf + w * 64 * RB;

  // A batch of up to 64 keys, lane l holding key l's K row (kr) and live bits (lv), their V
  // rows in the buffer rows set in bmask (in flight by DMA): scores, online softmax, P.V.
  auto consume = [&](const du4(&kr)[NC], uint32_t lv, uint64_t bmask) {
    float p[MQ];
#pragma unroll
    for (int i = 0; i < MQ; ++i) {
      p[i] = 0.f;
      if (i < nq) {
        float acc = 0.f;
#pragma unroll
        for (int cc = 0; cc < NC; ++cc)
          acc = Dec<T>::dot16(kr[cc], *reinterpret_cast<const du4*>(q_lds + i * RB + 16 * cc), acc);
        const float x = ((lv >> i) & 1u) ? acc * a.c : -INFINITY;
        const float mx = wave_max(x);
        if (mx != -INFINITY) {
          const float mn = fmaxf(m[i], mx);
          const float alpha = exp2f(m[i] - mn);
          m[i] = mn;
          p[i] = exp2f(x - mn);
          lsum[i] = lsum[i] * alpha + p[i];
#pragma unroll
          for (int d = 0; d < DPL; ++d) o[i][d] *= alpha;
        }
      }
    }
    // P.V, V from the buffer (this wave's own DMA: waiting for it is enough)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const char* vrow = vbuf_w + lane * DPL * ESZ;
    // eight rows at a time: their buffer rows are read together (a row outside bmask holds
    // stale data and is read but not used), so the reads' latency is paid once per eight
#pragma unroll
    for (int u0 = 0; u0 < 64; u0 += 8) {
      const uint32_t bits8 = (uint32_t)(bmask >> u0) & 0xffu;
      if (bits8 == 0u) continue;
      uint32_t vw[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (DPL * ESZ == 4)
          vw[e] = *reinterpret_cast<const uint32_t*>(vrow + (u0 + e) * RB);
        else
          vw[e] = *reinterpret_cast<const uint16_t*>(vrow + (u0 + e) * RB);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if ((bits8 >> e) & 1u) {
          float vx[DPL];
          vx[0] = Dec<T>::lo(vw[e]);
          if constexpr (DPL == 2) vx[DPL - 1] = Dec<T>::hi(vw[e]);
#pragma unroll
          for (int i = 0; i < MQ; ++i) {
            if (i < nq) {
              const float pk =
                  __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p[i]), u0 + e));
#pragma unroll
              for (int d = 0; d < DPL; ++d) o[i][d] = __builtin_fmaf(pk, vx[d], o[i][d]);
            }
          }
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // buffer reads done before the next DMA
  };

  if constexpr (LIST) {
    // The wave scans its blocks' keys for liveness and lists the live ones in LDS (kl_row:
    // the key's row in the head's cache, or -1 - j for the call's appended token j; kl_lv:
    // bit i set when the key is live for query i), then takes them 64 at a time: a block
    // with a few live keys costs its scan, not a round trip to memory.
    int nlist = 0;  // entries in the wave's list (at most 63 + 64)
    uint32_t g = (uint32_t)split;
    while (true) {
      while (nlist < 64 && g < n_groups) {
        const int cls = (int)(g / (uint32_t)a.groups);
        const int64_t b0 = (int64_t)(g - (uint32_t)cls * (uint32_t)a.groups) * 256 + 64 * w;
        const int64_t i1 = a.length > cls ? (a.length - 1 - cls) / a.s + 1 : 0;  // entries of the class
        g += (uint32_t)a.n_split;
        if (b0 >= i1) continue;
        const int64_t idx = b0 + lane;
        const int32_t t = (int32_t)(idx * a.s + cls);  // original position of this lane's key
        uint32_t bits = 0u;
        if (idx < i1) {
#pragma unroll
          for (int i = 0; i < MQ; ++i)
            if (i < nq && pred_live(a.pred, (int32_t)(a.qpos0 + i), t)) bits |= 1u << i;
        }
        const uint64_t any = __ballot(bits != 0u);
        if (any == 0ull) continue;
        if (bits) {
          const int pos = nlist + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(any >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)any, 0u));
          const int64_t jn = (int64_t)t - a.new_pos0;
          kl_row[w][pos] = (jn >= 0 && jn < a.n_new) ? (int32_t)(-1 - jn) : (int32_t)(cls * a.Q + idx);
          kl_lv[w][pos] = bits;
        }
        nlist += (int)__builtin_popcountll(any);
      }
      if (nlist == 0) break;
      const int nb = nlist < 64 ? nlist : 64;
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the list's entries are written
      int32_t code = 0;
      uint32_t lv = 0u;
      if (lane < nb) {
        code = kl_row[w][lane];
        lv = kl_lv[w][lane];
      }
      // the entries' V rows into buffer rows 0..nb-1 (RPI rows per DMA instruction, each
      // lane's row code read from the list; an appended row's 16-byte units from v_new),
      // and each entry's K row, one per lane, all in flight together
      const uint64_t newm = a.n_new ? __ballot(lane < nb && code < 0) : 0ull;
#pragma unroll
      for (int r = 0; r < 64 / RPI; ++r) {
        const int e = r * RPI + lane / LPR;
        const int32_t ce = kl_row[w][e];  // (past nb: not used)
        if (r * RPI < nb && e < nb && ce >= 0)
          lds_dma16_va(vbw + r * 1024, vh + (int64_t)ce * rowb + 16 * (lane % LPR));
      }
      if (newm) {
#pragma unroll
        for (int r = 0; r < 64 / RPI; ++r) {
          const int e = r * RPI + lane / LPR;
          const int32_t ce = __shfl(code, e);  // (every lane takes part in the shuffle)
          if ((newm >> e) & 1ull)
            *reinterpret_cast<du4*>(vbuf + w * 64 * RB + r * 1024 + 16 * lane) =
                *reinterpret_cast<const du4*>(vnew + (int64_t)(-1 - ce) * a.new_sn + 16 * (lane % LPR));
        }
      }
      du4 kr[NC];
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) kr[cc] = du4{0u, 0u, 0u, 0u};
      if (lane < nb) {
        const char* kp = code >= 0 ? kh + (int64_t)code * rowb : knew + (int64_t)(-1 - code) * a.new_sn;
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) kr[cc] = *reinterpret_cast<const du4*>(kp + 16 * cc);
      }
      consume(kr, lv, nb == 64 ? ~0ull : ((1ull << nb) - 1ull));
      // the list's entries past the batch move to its front
      nlist -= nb;
      if (nlist > 0) {
        int32_t r2 = 0;
        uint32_t l2 = 0u;
        if (lane < nlist) {
          r2 = kl_row[w][64 + lane];
          l2 = kl_lv[w][64 + lane];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane < nlist) {
          kl_row[w][lane] = r2;
          kl_lv[w][lane] = l2;
        }
      }
    }
  } else {
    // block by block: lane l scores key b0 + l of each of the wave's blocks that holds a
    // live key
    for (uint32_t g = (uint32_t)split; g < n_groups; g += (uint32_t)a.n_split) {
      const int cls = (int)(g / (uint32_t)a.groups);
      const int64_t b0 = (int64_t)(g - (uint32_t)cls * (uint32_t)a.groups) * 256 + 64 * w;
      const int64_t i1 = a.length > cls ? (a.length - 1 - cls) / a.s + 1 : 0;  // entries of the class
      if (b0 >= i1) continue;
      const char* kseg = kh + (int64_t)cls * a.Q * rowb;
      const char* vseg = vh + (int64_t)cls * a.Q * rowb;
      const int64_t idx = b0 + lane;
      const int32_t t = (int32_t)(idx * a.s + cls);  // original position of this lane's key
      uint32_t lv = 0u;  // bit i: (query i, key) is live
      if (idx < i1) {
#pragma unroll
        for (int i = 0; i < MQ; ++i)
          if (i < nq && pred_live(a.pred, (int32_t)(a.qpos0 + i), t)) lv |= 1u << i;
      }
      const uint64_t any = __ballot(lv != 0u);
      if (any == 0ull) continue;
      // keys appended by this call: read from k_new / v_new
      const int64_t jn = (int64_t)t - a.new_pos0;
      const bool isnew = idx < i1 && jn >= 0 && jn < a.n_new;
      const uint64_t newm = a.n_new ? __ballot(isnew) : 0ull;

      // the V rows of the keys live for some query, into this wave's buffer (lanes of a
      // dead row are masked off; a DMA instruction whose rows are all dead is skipped),
      // and the K row of each live key, one per lane, all in flight together
      const char* vblk = vseg + b0 * rowb;
#pragma unroll
      for (int r = 0; r < 64 / RPI; ++r) {
        if ((any >> (r * RPI)) & ((1ull << RPI) - 1ull)) {
          const int row = r * RPI + lane / LPR;
          if (((any & ~newm) >> row) & 1ull)
            lds_dma16(vbw + r * 1024, vblk, (uint32_t)(row * rowb + 16 * (lane % LPR)));
        }
      }
      if (newm & any) {
        // an appended row's 16-byte units, from v_new into the same place of the buffer
#pragma unroll
        for (int r = 0; r < 64 / RPI; ++r) {
          const int row = r * RPI + lane / LPR;
          if (((newm & any) >> row) & 1ull) {
            const int64_t jr = ((b0 + row) * a.s + cls) - a.new_pos0;
            *reinterpret_cast<du4*>(vbuf + w * 64 * RB + r * 1024 + 16 * lane) =
                *reinterpret_cast<const du4*>(vnew + jr * a.new_sn + 16 * (lane % LPR));
          }
        }
      }
      du4 kr[NC];
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) kr[cc] = du4{0u, 0u, 0u, 0u};
      if (lv) {
        const char* kp = isnew ? knew + jn * a.new_sn : kseg + idx * rowb;
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) kr[cc] = *reinterpret_cast<const du4*>(kp + 16 * cc);
      }
      consume(kr, lv, any);
    }
  }
  __syncthreads();  // every wave is past its buffer: it now holds the partials

  // the four waves' partials -> one normalised partial of the work-group
#pragma unroll
  for (int i = 0; i < MQ; ++i) {
    if (i < nq) {
      const float lt = wave_sum(lsum[i]);
      if (lane == 0) {
        red_m[w][i] = m[i];
        red_l[w][i] = lt;
      }
#pragma unroll
      for (int d = 0; d < DPL; ++d) red_o[w][i][lane * DPL + d] = o[i][d];
    }
  }
  __syncthreads();
  if (w == 0) {
    for (int i = 0; i < nq; ++i) {
      float M = red_m[0][i];
#pragma unroll
      for (int ww = 1; ww < kDecWaves; ++ww) M = fmaxf(M, red_m[ww][i]);
      float L = 0.f, acc[DPL];
#pragma unroll
      for (int d = 0; d < DPL; ++d) acc[d] = 0.f;
#pragma unroll
      for (int ww = 0; ww < kDecWaves; ++ww) {
        const float f = exp2f(red_m[ww][i] - M);
        L += f * red_l[ww][i];
#pragma unroll
        for (int d = 0; d < DPL; ++d) acc[d] += f * red_o[ww][i][lane * DPL + d];
      }
      const int64_t row = (bh * a.n_split + split) * nq + i;
      const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
      for (int d = 0; d < DPL; ++d) a.o_part[row * D + lane * DPL + d] = acc[d] * inv;
      if (lane == 0) a.lse_part[row] = L > 0.f ? (M + log2f(L)) * 0.69314718055994530942f : -INFINITY;
    }
  }
}

// o[bh, i] = sum_s exp(lse_s - M) o_s / sum_s exp(lse_s - M) over the splits; a row
// whose every partial is empty gives 0 and lse -inf.  One work-group per (bh, i): the
// weights are computed once into LDS, then 256 / D groups of D threads share the splits.
template <typename T>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* o_part, const float* lse_part, int n_split,
                                                           int nq, int D, char* o, int64_t o_sb, int64_t o_sn,
                                                           float* lse, int64_t lse_sb) {
  __shared__ float wts[kMergeMax];
  __shared__ float red[256];
  const int64_t bh = blockIdx.x / nq;
  const int i = blockIdx.x - (int)(bh * nq);
  const int tid = threadIdx.x;
  const float* lp = lse_part + bh * n_split * nq + i;
  float M = -INFINITY;
  for (int sp = tid; sp < n_split; sp += 256) {
    const float l = lp[(int64_t)sp * nq];
    wts[sp] = l;
    M = fmaxf(M, l);
  }
  red[tid] = M;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if (tid < h) red[tid] = fmaxf(red[tid], red[tid + h]);
    __syncthreads();
  }
  M = red[0];
  __syncthreads();
  float den = 0.f;
  for (int sp = tid; sp < n_split; sp += 256) {
    const float l = wts[sp];
    const float f = (M == -INFINITY || l == -INFINITY) ? 0.f : expf(l - M);
    wts[sp] = f;
    den += f;
  }
  red[tid] = den;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if (tid < h) red[tid] += red[tid + h];
    __syncthreads();
  }
  den = red[0];
  __syncthreads();
  const int parts = 256 / D;
  const int d = tid % D, part = tid / D;
  float num = 0.f;
  if (part < parts) {
    // (an empty split's partial is 0 and its weight 0: no branch in the loop)
    const float* op = o_part + (bh * n_split * nq + i) * D + d;
#pragma unroll 8
    for (int sp = part; sp < n_split; sp += parts) num = __builtin_fmaf(wts[sp], op[(int64_t)sp * nq * D], num);
  }
  red[tid] = num;
  __syncthreads();
  if (tid < D) {
    for (int pp = 1; pp < parts; ++pp) num += red[pp * D + tid];
    const float v = den > 0.f ? num / den : 0.f;
    *reinterpret_cast<T*>(o + ((bh * o_sb + (int64_t)i * o_sn) * (int64_t)sizeof(T)) + tid * (int64_t)sizeof(T)) = (T)v;
  }
  if (lse && tid == 0) lse[bh * lse_sb + i] = den > 0.f ? M + logf(den) : -INFINITY;
}

// Rows of the new tokens into their basis rows: unit u of row j of head bh of tensor
// (K, V), 16- or 4-byte units.
template <int VB>
__global__ __launch_bounds__(256) void kv_append_kernel(const char* k_new, const char* v_new, int64_t n_sb,
                                                        int64_t n_sn, char* kc, char* vc, int64_t c_sb,
                                                        int64_t c_sn, int64_t BH, int64_t n, int32_t upr,
                                                        int64_t pos0, int32_t s, int64_t Q) {
  typedef uint32_t unit __attribute__((ext_vector_type(VB / 4)));
  const int64_t total = 2 * BH * n * upr;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (int64_t)gridDim.x * blockDim.x) {
    const int64_t u = g % upr;
    int64_t r = g / upr;
    const int64_t j = r % n;
    r /= n;
    const int64_t bh = r % BH;
    const bool is_v = r >= BH;
    const int64_t t = pos0 + j;
    const int64_t row = (t % s) * Q + t / s;
    const char* src = (is_v ? v_new : k_new) + bh * n_sb + j * n_sn + u * VB;
    char* dst = (is_v ? vc : kc) + bh * c_sb + row * c_sn + u * VB;
    *reinterpret_cast<unit*>(dst) = *reinterpret_cast<const unit*>(src);
  }
}

struct Plan {
  int32_t s, n_split;
  int64_t groups, Q;
};

// Split of the keys: each class's segment in groups of 256 entries, the groups of a head
// numbered class-major and dealt round-robin to n_split work-groups per head, about
// kDecTarget work-groups in all and at most one per group that holds entries.  With s > 1
// a class takes `groups` numbers, at least as many as the longest segment needs and with
// no factor in common with n_split (the surplus numbers are empty groups), so the groups at
// one place of every class, such as a window's last entries, go to different work-groups.
// n_split <= kDecTarget = kMergeMax, the splits the merge holds in LDS.
Plan plan_of(int64_t BH, int64_t capacity, int64_t length, int32_t residue_s) {
  Plan p;
  p.s = residue_s > 1 ? residue_s : 1;
  p.Q = capacity / p.s;
  const int64_t cnt_max = (length + p.s - 1) / p.s;
  const int64_t need = (cnt_max + 255) / 256;
  int64_t per = (kDecTarget + BH - 1) / BH;
  if (per > p.s * need) per = p.s * need;
  p.n_split = (int32_t)per;
  p.groups = need;
  if (p.s > 1 && per > 1)
    while (std::gcd(p.groups, per) != 1) ++p.groups;  // ends within per steps (per and per+1 are coprime)
  return p;
}

int check_decode(const pa_decode_args* x) {
  PA_CHECK_ARG(x, "pa_decode: null arguments");
  PA_CHECK_ARG(x->BH >= 1 && x->BH <= 65535, "pa_decode: BH=%lld not in 1..65535", (long long)x->BH);
  PA_CHECK_ARG(x->nq >= 1 && x->nq <= kDecMaxQ, "pa_decode: nq=%d not in 1..%d", x->nq, kDecMaxQ);
  PA_CHECK_ARG(x->dtype == PA_BF16 || x->dtype == PA_F16 || x->dtype == PA_F32, "pa_decode: dtype %d", x->dtype);
  PA_CHECK_ARG(x->D == 128 || x->D == 64, "pa_decode: D=%d (64 or 128)", x->D);
  PA_CHECK_ARG(x->dtype != PA_F32 || x->D == 64, "pa_decode: float32 needs D = 64");
  const int32_t s = x->residue_s > 1 ? x->residue_s : 1;
  PA_CHECK_ARG(s <= kMaxResidue, "pa_decode: residue_s=%d exceeds %d classes", s, kMaxResidue);
  PA_CHECK_ARG(x->capacity >= 1 && x->capacity < (1ll << 31) && x->capacity % s == 0,
               "pa_decode: capacity=%lld must be in 1..2^31-1 and a multiple of s=%d", (long long)x->capacity, s);
  PA_CHECK_ARG(x->length >= 0 && x->length <= x->capacity, "pa_decode: length=%lld outside 0..capacity",
               (long long)x->length);
  PA_CHECK_ARG(x->qpos0 >= 0 && x->qpos0 + x->nq <= (1ll << 31), "pa_decode: query positions out of range");
  PA_CHECK_ARG(!x->mask.perm_q && !x->mask.perm_kv,
               "pa_decode: the cache's basis is residue_s; the mask takes no permutation tables");
  const int rc = check_mask(&x->mask, x->capacity > x->qpos0 + x->nq ? x->capacity : x->qpos0 + x->nq);
  if (rc) return rc;
  PA_CHECK_ARG(x->q && x->k_cache && x->v_cache && x->o, "pa_decode: null q / cache / o");
  const int esz = x->dtype == PA_F32 ? 4 : 2;
  auto al = [&](const void* ptr, int64_t sb, int64_t sn) {
    return (reinterpret_cast<uintptr_t>(ptr) % 16) == 0 && (sb * esz) % 16 == 0 && (sn * esz) % 16 == 0;
  };
  PA_CHECK_ARG(al(x->q, x->q_sb, x->q_sn) && al(x->k_cache, x->c_sb, x->c_sn) && al(x->v_cache, x->c_sb, x->c_sn),
               "pa_decode: q and cache rows must be 16-byte aligned");
  PA_CHECK_ARG(x->c_sn >= x->D && x->q_sn >= x->D, "pa_decode: row strides below D");
  PA_CHECK_ARG(x->n_new >= 0 && x->n_new <= kDecMaxQ, "pa_decode: n_new=%lld not in 0..%d", (long long)x->n_new,
               kDecMaxQ);
  if (x->n_new > 0) {
    PA_CHECK_ARG(x->k_new && x->v_new, "pa_decode: null k_new / v_new");
    PA_CHECK_ARG(al(x->k_new, x->new_sb, x->new_sn) && al(x->v_new, x->new_sb, x->new_sn),
                 "pa_decode: k_new / v_new rows must be 16-byte aligned");
    PA_CHECK_ARG(x->new_sn >= x->D, "pa_decode: new_sn below D");
    PA_CHECK_ARG(x->new_pos0 >= 0 && x->new_pos0 + x->n_new <= x->length,
                 "pa_decode: appended positions %lld..%lld outside the attended length %lld",
                 (long long)x->new_pos0, (long long)(x->new_pos0 + x->n_new), (long long)x->length);
  }
  return PA_OK;
}

// The identity basis takes the kernel's key list (live keys spread thinly over many
// blocks); a residue basis, whose relabelling gathers the live keys into few full blocks,
// takes block by block.
template <typename T, int D>
int launch_decode(const DecK& k, int64_t BH, hipStream_t s) {
  const dim3 grid((unsigned)k.n_split, (unsigned)BH);
  if (k.nq == 1) {
    if (k.s == 1)
      hipLaunchKernelGGL((decode_kernel<T, D, 1, true>), grid, dim3(256), 0, s, k);
    else
      hipLaunchKernelGGL((decode_kernel<T, D, 1, false>), grid, dim3(256), 0, s, k);
  } else {
    if (k.s == 1)
      hipLaunchKernelGGL((decode_kernel<T, D, kDecMaxQ, true>), grid, dim3(256), 0, s, k);
    else
      hipLaunchKernelGGL((decode_kernel<T, D, kDecMaxQ, false>), grid, dim3(256), 0, s, k);
  }
  PA_LAUNCH_CHECK("decode_kernel");
  return PA_OK;
}

}  // namespace
}  // namespace pa

extern "C" int pa_decode_workspace(const pa_decode_args* x, int64_t* bytes) {
  const int rc = pa::check_decode(x);
  if (rc) return rc;
  PA_CHECK_ARG(bytes, "pa_decode_workspace: null output");
  const pa::Plan p = pa::plan_of(x->BH, x->capacity, x->length, x->residue_s);
  *bytes = x->BH * (int64_t)p.n_split * x->nq * (x->D + 1) * 4;
  return PA_OK;
}

// The partials of one pa_decode_fwd_static call: a per-device global of the library, so
// the call allocates nothing.  Host code never passes `scratch` itself (on the host the
// name is only a stand-in for the symbol): its device address on the current device
// comes from hipGetSymbolAddress, once per device, in decode_scratch.
constexpr int64_t kDecodeScratchBytes = 8ll << 20;
static __device__ __align__(256) float scratch[kDecodeScratchBytes / 4];

namespace pa {
namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kScratchDevices] = {};

// The device address of `scratch` on the current device (looked up on the first call
// on that device, then kept).
int decode_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  PA_CHECK_ARG(dev >= 0 && dev < kScratchDevices, "pa_decode_fwd_static: device %d beyond %d", dev,
               kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    PA_CHECK_ARG(ptr != nullptr, "pa_decode_fwd_static: no device address for the scratch array");
    g_scratch[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch[dev];
  return PA_OK;
}

int decode_launch(const pa_decode_args* x, const Plan& p, float* ws, hipStream_t s);

}  // namespace
}  // namespace pa

extern "C" int pa_decode_fwd(const pa_decode_args* x, void* stream) {
  const int rc = pa::check_decode(x);
  if (rc) return rc;
  const pa::Plan p = pa::plan_of(x->BH, x->capacity, x->length, x->residue_s);
  const int64_t need = x->BH * (int64_t)p.n_split * x->nq * (x->D + 1) * 4;
  PA_CHECK_ARG(p.n_split == 0 || (x->workspace && x->workspace_bytes >= need &&
                                  (reinterpret_cast<uintptr_t>(x->workspace) % 16) == 0),
               "pa_decode_fwd: workspace of %lld bytes (16-byte aligned) needed, got %lld", (long long)need,
               (long long)x->workspace_bytes);
  return pa::decode_launch(x, p, static_cast<float*>(x->workspace), static_cast<hipStream_t>(stream));
}

extern "C" int pa_decode_fwd_static(const pa_decode_args* x, void* stream) {
  const int rc = pa::check_decode(x);
  if (rc) return rc;
  PA_CHECK_ARG(!x->workspace && x->workspace_bytes == 0,
               "pa_decode_fwd_static: takes no workspace (the partials go to the library's scratch)");
  const pa::Plan p = pa::plan_of(x->BH, x->capacity, x->length, x->residue_s);
  const int64_t need = x->BH * (int64_t)p.n_split * x->nq * (x->D + 1) * 4;
  PA_CHECK_ARG(need <= kDecodeScratchBytes,
               "pa_decode_fwd_static: the split partials need %lld bytes, more than the %lld-byte scratch "
               "(call pa_decode_fwd with a workspace)",
               (long long)need, (long long)kDecodeScratchBytes);
  float* ws = nullptr;
  if (p.n_split > 0) {
    if (int r = pa::decode_scratch(&ws)) return r;
  }
  return pa::decode_launch(x, p, ws, static_cast<hipStream_t>(stream));
}

namespace pa {
namespace {

int decode_launch(const pa_decode_args* x, const Plan& p, float* ws, hipStream_t s) {
  pa::DecK k;
  k.q = static_cast<const char*>(x->q);
  k.q_sb = x->q_sb;
  k.q_sn = x->q_sn;
  k.k = static_cast<char*>(x->k_cache);
  k.v = static_cast<char*>(x->v_cache);
  k.c_sb = x->c_sb;
  k.c_sn = x->c_sn;
  k.qpos0 = x->qpos0;
  k.length = x->length;
  k.Q = p.Q;
  k.groups = p.groups;
  k.nq = x->nq;
  k.s = p.s;
  k.n_split = p.n_split;
  k.c = (x->scale > 0.f ? x->scale : 1.f / sqrtf((float)x->D)) * 1.4426950408889634f;
  k.pred = pa::make_pred(x->mask);
  k.o_part = ws;
  k.lse_part = ws ? ws + x->BH * (int64_t)p.n_split * x->nq * x->D : nullptr;
  const int64_t esz = x->dtype == PA_F32 ? 4 : 2;
  k.n_new = x->n_new;
  k.new_pos0 = x->new_pos0;
  k.k_new = x->n_new ? static_cast<const char*>(x->k_new) : nullptr;
  k.v_new = x->n_new ? static_cast<const char*>(x->v_new) : nullptr;
  k.new_sb = x->n_new ? x->new_sb * esz : 0;
  k.new_sn = x->n_new ? x->new_sn * esz : 0;
  if (p.n_split > 0) {
    int r = PA_OK;
    if (x->dtype == PA_BF16)
      r = x->D == 128 ? pa::launch_decode<__bf16, 128>(k, x->BH, s) : pa::launch_decode<__bf16, 64>(k, x->BH, s);
    else if (x->dtype == PA_F16)
      r = x->D == 128 ? pa::launch_decode<_Float16, 128>(k, x->BH, s) : pa::launch_decode<_Float16, 64>(k, x->BH, s);
    else
      r = pa::launch_decode<float, 64>(k, x->BH, s);
    if (r) return r;
  }
  const unsigned g = (unsigned)(x->BH * x->nq);
  char* o = static_cast<char*>(x->o);
#define PA_MERGE(TT)                                                                                            \
  hipLaunchKernelGGL((pa::decode_merge_kernel<TT>), dim3(g), dim3(256), 0, s, k.o_part, k.lse_part, p.n_split,  \
                     x->nq, x->D, o, x->o_sb, x->o_sn, x->lse, x->lse_sb)
  if (x->dtype == PA_BF16)
    PA_MERGE(__bf16);
  else if (x->dtype == PA_F16)
    PA_MERGE(_Float16);
  else
    PA_MERGE(float);
#undef PA_MERGE
  PA_LAUNCH_CHECK("decode_merge_kernel");
  return PA_OK;
}

}  // namespace
}  // namespace pa

extern "C" int pa_kv_append(const void* k_new, const void* v_new, int64_t new_sb, int64_t new_sn, void* k_cache,
                            void* v_cache, int64_t c_sb, int64_t c_sn, int64_t BH, int64_t n, int32_t D,
                            int32_t dtype, int64_t capacity, int64_t pos0, int32_t residue_s, void* stream) {
  PA_CHECK_ARG(dtype == PA_BF16 || dtype == PA_F16 || dtype == PA_F32, "pa_kv_append: dtype %d", dtype);
  const int64_t s = residue_s > 1 ? residue_s : 1;
  PA_CHECK_ARG(s <= pa::kMaxResidue, "pa_kv_append: residue_s=%d exceeds %d classes", residue_s, pa::kMaxResidue);
  PA_CHECK_ARG(BH >= 1 && n >= 0 && D >= 1, "pa_kv_append: BH=%lld n=%lld D=%d", (long long)BH, (long long)n, D);
  PA_CHECK_ARG(capacity >= 1 && capacity % s == 0, "pa_kv_append: capacity=%lld not a multiple of s=%lld",
               (long long)capacity, (long long)s);
  PA_CHECK_ARG(pos0 >= 0 && pos0 + n <= capacity, "pa_kv_append: positions %lld..%lld exceed capacity %lld",
               (long long)pos0, (long long)(pos0 + n), (long long)capacity);
  if (n == 0) return PA_OK;
  PA_CHECK_ARG(k_new && v_new && k_cache && v_cache, "pa_kv_append: null pointer");
  const int esz = dtype == PA_F32 ? 4 : 2;
  const int64_t rb = (int64_t)D * esz;
  PA_CHECK_ARG(rb % 4 == 0, "pa_kv_append: row bytes %lld not a multiple of 4", (long long)rb);
  PA_CHECK_ARG(c_sn >= D && new_sn >= D, "pa_kv_append: row strides below D");
  auto al = [](const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; };
  const bool v16 = rb % 16 == 0 && al(k_new, 16) && al(v_new, 16) && al(k_cache, 16) && al(v_cache, 16) &&
                   (new_sb * esz) % 16 == 0 && (new_sn * esz) % 16 == 0 && (c_sb * esz) % 16 == 0 &&
                   (c_sn * esz) % 16 == 0;
  PA_CHECK_ARG(v16 || (al(k_new, 4) && al(v_new, 4) && al(k_cache, 4) && al(v_cache, 4)),
               "pa_kv_append: pointers must be 4-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int VB = v16 ? 16 : 4;
  const int32_t upr = (int32_t)(rb / VB);
  int64_t blocks = (2 * BH * n * upr + 255) / 256;
  if (blocks > (1 << 20)) blocks = 1 << 20;
  const char* kn = static_cast<const char*>(k_new);
  const char* vn = static_cast<const char*>(v_new);
  char* kc = static_cast<char*>(k_cache);
  char* vc = static_cast<char*>(v_cache);
  if (v16)
    hipLaunchKernelGGL(pa::kv_append_kernel<16>, dim3((unsigned)blocks), dim3(256), 0, st, kn, vn, new_sb * esz,
                       new_sn * esz, kc, vc, c_sb * esz, c_sn * esz, BH, n, upr, pos0, (int32_t)s, capacity / s);
  else
    hipLaunchKernelGGL(pa::kv_append_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, st, kn, vn, new_sb * esz,
                       new_sn * esz, kc, vc, c_sb * esz, c_sn * esz, BH, n, upr, pos0, (int32_t)s, capacity / s);
  PA_LAUNCH_CHECK("kv_append_kernel");
  return PA_OK;
}
