// Ragged joint prefill + decode GQA attention on gfx950 (fp16 or int8 KV).
//
// Semantics follow the reference host loop (examples/intfer_cli/main.cpp:
// 7657-7701): per row and q head, s_t = (q . k_t) / sqrt(hd) over the
// sequence's KV positions t <= pos, softmax, o = sum_t p_t v_t.  Prefill and
// verify rows of a sequence see the rows before them in the same chunk,
// because KV is appended for every row before attention runs.
//
// Work decomposition: the pack kernel emits units (sequence, kv head, q-block
// of up to 8 tokens, KV split).  One wave runs one unit: the q-block's
// tokens x the GQA group (2 heads) form the 16 columns of S^T = K Q^T and of
// O^T = V^T P^T, so K is the MFMA A operand row-major and V is read from its
// transposed page; each 32-token page is one step with wave-level online
// softmax (base-2 exponent).  Partial (m, l, O) per unit are merged by the
// combine kernel, which also emits the per-token int8 input of the O
// projection.  Decode units use 2 of the 16 columns; the kernel is bound by
// the KV stream, which is read exactly once per unit.
#include "ifr_dev.h"
#include "ifr_kernels.h"

namespace ifrk {
namespace {

constexpr int kHD = 128;
constexpr int kPage = 32;

// One lane's W dwords of a K or V fragment.  fp16 pages (16 bytes a lane)
// are a streaming read (each page of a decode or verify unit is read once):
// c64 decode rows 62.4 -> 59.9 us (bench.py --attn-sweep); the 8-byte int8
// fragments were slower that way and keep plain loads.
template <int W>
__device__ __forceinline__ void load_frag(const uint32_t* src, uint32_t (&dst)[W]) {
  if constexpr (W == 4) {
    const v4i x = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(src));
    dst[0] = (uint32_t)x.x; dst[1] = (uint32_t)x.y; dst[2] = (uint32_t)x.z; dst[3] = (uint32_t)x.w;
  } else {
#pragma unroll
    for (int q = 0; q < W; ++q) dst[q] = src[q];
  }
}

template <bool KV8, int NT>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs p, KVLayout kv) {
  const int lane = threadIdx.x & 63;
  // wave-uniform unit index: the unit record and block-table entries become
  // scalar loads, which do not queue behind the vector K/V loads
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Dispatch order: the dense workgroups (slots [n_shared, n_slots)) take the
  // first block ids, the chunked region the rest.  The dense units stream KV
  // from HBM and the chunked ones are bound by MFMA / VALU issue; started
  // first, the dense units keep HBM busy while the chunked workgroups fill
  // the remaining slots, instead of queueing behind them (c64 decode rows +
  // a 512-row chunk: 81.3 -> 73.6 us).  Only the order changes, not the work.
  const int nsw = p.n_shared / 4, nwg = (int)gridDim.x, ndw = nwg - nsw;
  const int bid = (int)blockIdx.x < ndw ? nsw + (int)blockIdx.x : (int)blockIdx.x - ndw;
  const int slot = bid * 4 + w;
  // Workgroups of the chunked region serve 4 q-blocks of one sequence with the
  // same kv head and split: they stream each K/V page once into LDS and all 4
  // waves read it there.  Other workgroups run 4 independent units.
  // (fp16 pages only: the host rejects n_shared > 0 for int8 KV)
  const bool shared = !KV8 && bid * 4 < p.n_shared;  // workgroup-uniform
  if (!shared && slot >= p.n_slots) return;         // (no barrier on this path)
  const int u = p.order[slot];
  if (!shared && u < 0) return;
  // In a shared workgroup an idle wave (u < 0) still loads and synchronizes;
  // it borrows the unit of the chunk's last q-block (always present), whose
  // KV range covers the others'.
  int u_pg = u;
  if (shared) {
#pragma unroll
    for (int q = 3; q >= 0; --q) {
      const int uq = p.order[bid * 4 + q];
      if (uq >= 0) { u_pg = uq; break; }
    }
  }
  const bool active = u >= 0;
  const AttnUnit un = p.units[active ? u : u_pg];
  const AttnUnit upg = p.units[u_pg];
  const int G = p.nq / kv.nkv;
  const int rows = un.qn * G;  // valid columns of the unit's NT x 16 column tiles
  const int c = lane & 15, g = lane >> 4;
  bool colv[NT];
  int qpos[NT];
  // Q^T as the B operand: column tile t, MFMA i covers dims 32i + 8g .. +8 of
  // column 16t + c = (q token, head of the GQA group).
  v8h qf[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int col = 16 * t + c;
    colv[t] = active && col < rows;
    const int qtok = col / G, qj = col % G;
    qpos[t] = un.qpos0 + qtok;
    if (colv[t]) {
      const _Float16* qp = reinterpret_cast<const _Float16*>(p.q) +
                           ((size_t)(un.row0 + qtok) * p.nq + un.kvh * G + qj) * kHD + 8 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) qf[t][i] = *reinterpret_cast<const v8h*>(qp + 32 * i);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) qf[t][i] = (v8h){0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  float m_run[NT], l_run[NT];
  v4f o[NT][8];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    m_run[t] = -INFINITY;
    l_run[t] = 0.0f;
#pragma unroll
    for (int d = 0; d < 8; ++d) o[t][d] = (v4f){0.f, 0.f, 0.f, 0.f};
  }

  const int32_t* bt = kv.block_table + (size_t)un.seq * kv.max_pages;
  // One page = 32 tokens.  Raw K/V fragments of a page (fp16, or int8 with
  // per-token scales); two buffers alternate so the next page's loads are in
  // flight while the current page is computed.  Every load is unconditional
  // (the page index is clamped to the unit's last page), so the wait before a
  // page covers only that page's loads.
  struct PageBuf {
    uint32_t k[2][4][KV8 ? 2 : 4];  // K tile h, k-step i: 8 dims of token 2c + h
    uint32_t v[8][KV8 ? 2 : 4];     // V^T tile d: 8 tokens of dim 16d + c
    uint16_t ks[2][4], vs[8];
  };
  // pages are [kv_lo + 32 i, +32); a shared workgroup walks its widest range
  const int last = ((shared ? upg.kv_hi : un.kv_hi) - 1 - un.kv_lo) / kPage;
  // fragment-major pages: fragment f is 64 lanes x 8 elements, lane at 8 * lane
  constexpr int W = KV8 ? 2 : 4;
  auto page_of = [&](int i) {
    const int t0 = un.kv_lo + kPage * min(i, last);
    return (size_t)bt[t0 / kPage] * kv.nkv + un.kvh;
  };
  auto load_k = [&](PageBuf& b, int i) {
    const size_t pb = page_of(i);
    const uint8_t* kp = reinterpret_cast<const uint8_t*>(kv.kpool) + pb * kPage * kHD * (KV8 ? 1 : 2);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const size_t e = (size_t)((h * 4 + i4) * 64 + lane) * 8;  // element index
        const uint32_t* src = reinterpret_cast<const uint32_t*>(kp + e * (KV8 ? 1 : 2));
        load_frag<W>(src, b.k[h][i4]);
      }
    if constexpr (KV8) {
      const uint16_t* ksc = kv.kscale + pb * kPage;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) b.ks[h][r] = ksc[8 * g + 2 * r + h];
    }
  };
  auto load_v = [&](PageBuf& b, int i) {
    const size_t pb = page_of(i);
    const uint8_t* vp = reinterpret_cast<const uint8_t*>(kv.vpool) + pb * kHD * kPage * (KV8 ? 1 : 2);
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const size_t e = (size_t)(d * 64 + lane) * 8;
      const uint32_t* src = reinterpret_cast<const uint32_t*>(vp + e * (KV8 ? 1 : 2));
      load_frag<W>(src, b.v[d]);
    }
    if constexpr (KV8) {
      const uint16_t* vsc = kv.vscale + pb * kPage;
#pragma unroll
      for (int j = 0; j < 8; ++j) b.vs[j] = vsc[8 * g + j];
    }
  };
  auto frag = [&](const uint32_t* w) -> v8h {  // 8 fp16 from raw fp16 or int8
    v8h f;
    if constexpr (!KV8) {
      f = __builtin_bit_cast(v8h, (v4i){(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
    } else {
      // int8 b -> fp16 exactly: byte b ^ 0x80 = b + 128 under the exponent
      // byte 0x64 is the half 1024 + (b + 128); subtracting 1152 leaves b.
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t u = w[q] ^ 0x80808080u;
        const h2 lo = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
        const h2 hi = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
        f[4 * q + 0] = lo[0];
        f[4 * q + 1] = lo[1];
        f[4 * q + 2] = hi[0];
        f[4 * q + 3] = hi[1];
      }
    }
    return f;
  };
  // K fragments and scales from kb, V fragments and scales from vb
  auto step = [&](const PageBuf& kb, const PageBuf& vb, int i) {
    const int t0 = un.kv_lo + kPage * i;
    // ---- S^T: K tile h covers tokens 2c' + h; lane (c, g) reg r -> token 8g + 2r + h.
    v8h kf[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) kf[h][i4] = frag(kb.k[h][i4]);
    v8h phi[NT], plo[NT];
    float alpha[NT];
    // A page wholly below the unit's first query position and its KV end
    // masks nothing for a valid column (columns past the unit's rows carry
    // q = 0, finite scores, and are never stored), so only boundary pages
    // pay for the mask.  Wave-uniform.
    const bool interior = t0 + kPage - 1 <= un.qpos0 && t0 + kPage <= un.kv_hi;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      v4f s[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        s[h] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
          s[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[h][i4], qf[t][i4], s[h], 0, 0, 0);
      }
      float sv[8];
      float mt = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int tk = t0 + 8 * g + 2 * r + h;
          float v = s[h][r];
          if constexpr (KV8) v *= ifrd::h2f(kb.ks[h][r]);
          v *= p.scale_log2;
          if (!interior && (!colv[t] || tk > qpos[t] || tk >= un.kv_hi)) v = -INFINITY;
          sv[2 * r + h] = v;
          mt = fmaxf(mt, v);
        }
      // the 4 lane groups hold the page's other tokens: exchange through the
      // gfx950 lane swaps (VALU), not the LDS crossbar; same partner values
      mt = fmaxf(mt, ifrd::lane_xor<16>(mt));
      mt = fmaxf(mt, ifrd::lane_xor<32>(mt));
      const float m_new = fmaxf(m_run[t], mt);
      const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
      alpha[t] = __builtin_amdgcn_exp2f(m_run[t] - m_use);
      // P enters the PV product as an fp16 hi + lo pair (p ~ hi + lo to ~22
      // bits): V is exact in fp16, so O carries fp32-level accuracy and the
      // downstream per-token int8 codes match the fp32 reference loop.
      float rs = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float pf = __builtin_amdgcn_exp2f(sv[j] - m_use);
        rs += pf;
        const float pv = KV8 ? pf * ifrd::h2f(vb.vs[j]) : pf;
        const _Float16 hh = (_Float16)pv;
        phi[t][j] = hh;
        plo[t][j] = (_Float16)(pv - (float)hh);
      }
      rs += ifrd::lane_xor<16>(rs);
      rs += ifrd::lane_xor<32>(rs);
      l_run[t] = l_run[t] * alpha[t] + rs;
      m_run[t] = m_new;
    }
    // rescale O only when some column's running max moved (x * 1 is exact)
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (!__all(alpha[t] == 1.0f))
#pragma unroll
        for (int d = 0; d < 8; ++d) o[t][d] *= alpha[t];
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const v8h vf = frag(vb.v[d]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        o[t][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, phi[t], o[t][d], 0, 0, 0);
        o[t][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, plo[t], o[t][d], 0, 0, 0);
      }
    }
  };
  if (shared) {
   if constexpr (!KV8) {
    // fp16 pages only (the host sets n_shared = 0 for int8 KV).  LDS holds two
    // pages of 16 fragments (8 K, 8 V) x 64 lanes x 16 bytes; wave w stages
    // fragments 4w..4w+3.  One barrier per page: page i is stored into buffer
    // i & 1, and every wave has finished page i - 1 (the other buffer's
    // previous content) before anyone passes the barrier of page i.
    __shared__ uint4 kvs[2][16][64];
    // waves 0-1 stage K fragments 4w..4w+3 (h * 4 + i), waves 2-3 V fragments (d)
    const uint8_t* kvbase = reinterpret_cast<const uint8_t*>(w < 2 ? kv.kpool : kv.vpool);
    const int f0 = w < 2 ? 4 * w : 4 * w - 8;
    auto src_of = [&](int i) {
      const int t0 = un.kv_lo + kPage * min(i, last);
      const size_t pb = (size_t)bt[t0 / kPage] * kv.nkv + un.kvh;
      return reinterpret_cast<const uint4*>(kvbase) + pb * (kPage * kHD / 8) + (size_t)f0 * 64 + lane;
    };
    const uint4* sp = src_of(0);
    uint4 s0 = sp[0], s1 = sp[64], s2 = sp[128], s3 = sp[192];
    for (int i = 0;; ++i) {
      uint4* dst = &kvs[i & 1][4 * w][lane];
      dst[0] = s0;
      dst[64] = s1;
      dst[128] = s2;
      dst[192] = s3;
      sp = src_of(i + 1);
      s0 = sp[0];
      s1 = sp[64];
      s2 = sp[128];
      s3 = sp[192];
      __syncthreads();
      if (active) {
        PageBuf b;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            const uint4 x = kvs[i & 1][h * 4 + i4][lane];
            b.k[h][i4][0] = x.x; b.k[h][i4][1] = x.y; b.k[h][i4][2] = x.z; b.k[h][i4][3] = x.w;
          }
#pragma unroll
        for (int d = 0; d < 8; ++d) {
          const uint4 x = kvs[i & 1][8 + d][lane];
          b.v[d][0] = x.x; b.v[d][1] = x.y; b.v[d][2] = x.z; b.v[d][3] = x.w;
        }
        step(b, b, i);
      }
      if (i >= last) break;
    }
   }
  } else {
    // K double-buffered, V single: page i + 1's K loads are in flight
    // while page i is computed, its V loads once page i's PV product has
    // read V(i) (during page i + 1's scores and softmax)
    PageBuf kA, kB, vb;
    load_k(kA, 0);
    load_v(vb, 0);
    for (int i = 0;; i += 2) {
      load_k(kB, i + 1);
      step(kA, vb, i);
      load_v(vb, i + 1);
      if (i + 1 > last) break;
      load_k(kA, i + 2);
      step(kB, vb, i + 1);
      load_v(vb, i + 2);
      if (i + 2 > last) break;
    }
  }
  if (!active) return;
  // ---- partials: O^T lane (c, g) reg r -> dim 16d + 4g + r of column 16t + c.
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (!colv[t]) continue;
    const size_t pc = (size_t)u * 16 * NT + 16 * t + c;
    float* po = p.part_o + pc * kHD;
#pragma unroll
    for (int d = 0; d < 8; ++d)
      *reinterpret_cast<v4f*>(po + 16 * d + 4 * g) = o[t][d];
    if (g == 0) {
      p.part_ml[pc * 2 + 0] = m_run[t];
      p.part_ml[pc * 2 + 1] = l_run[t];
    }
  }
}

// Merge the KV-split partials of one row for all heads, then per-token int8
// quantization (half-away) of the [nq*hd] attention row for the O projection.
// Thread t owns the CS consecutive dims [CS t, CS t + CS) of the row (CS a
// power of two dividing hd, so a chunk never straddles a head; threads past
// nq*hd/CS idle).  The merge runs the splits in order: the max over all
// splits first, then l and O accumulated split by split, loaded in rounds of
// 4 with clamped (unconditional) indices so each round is one memory latency.
template <int CS>
__device__ __forceinline__ int group_sum_int(int v) {
  // the 128 columns of one K group are 128 / CS consecutive lanes
  if constexpr (CS == 8) {
    return ifrd::row16_sum_int(v);
  } else {
    v += __builtin_bit_cast(int, ifrd::lane_xor<1>(__builtin_bit_cast(float, v)));
    v += __builtin_bit_cast(int, ifrd::lane_xor<2>(__builtin_bit_cast(float, v)));
    if constexpr (CS == 16) v += __builtin_bit_cast(int, ifrd::lane_xor<4>(__builtin_bit_cast(float, v)));
    return v;
  }
}

template <int CS>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
  const int m = blockIdx.x;
  const int N = a.nq * a.hd;
  const int G = a.nq / a.nkv;
  const bool own = (int)threadIdx.x * CS < N;
  const int e0 = own ? threadIdx.x * CS : 0;
  const int h = e0 / a.hd, d0 = e0 % a.hd;
  const int kvh = h / G, j = h % G;
  const int ns = a.comb_nsplit[m];
  const int base = a.comb_base[m] + kvh * ns;
  const int col = a.comb_tok[m] * G + j;
  // the output gate's CS fp16 values (issued first; used after the merge)
  uint32_t gw[CS / 2];
  if (a.gate) {
    const uint4* gp = reinterpret_cast<const uint4*>(a.gate + (size_t)m * N + e0);
#pragma unroll
    for (int r = 0; r < CS / 8; ++r) {
      const uint4 x = gp[r];
      gw[4 * r] = x.x; gw[4 * r + 1] = x.y; gw[4 * r + 2] = x.z; gw[4 * r + 3] = x.w;
    }
  }
  float mx = -INFINITY;
  float L = 0.0f;
  float acc[CS];
#pragma unroll
  for (int i = 0; i < CS; ++i) acc[i] = 0.0f;
  const float2* ml2 = reinterpret_cast<const float2*>(a.part_ml);
  // Up to R1 splits: one round of loads, the max taken from the loaded
  // (m, l) pairs; more: a max pass, then the weighted sum.  Either way the
  // splits are summed in ascending order with the same operands.
  constexpr int R1 = CS == 8 ? 8 : 4;
  if (ns <= R1) {
    float2 mlv[R1];
    float4 ov[R1][CS / 4];
#pragma unroll
    for (int q = 0; q < R1; ++q) {
      const size_t pi = (size_t)(base + min(q, ns - 1)) * a.ucols + col;
      mlv[q] = ml2[pi];
      const float4* po = reinterpret_cast<const float4*>(a.part_o + pi * a.hd + d0);
#pragma unroll
      for (int r = 0; r < CS / 4; ++r) ov[q][r] = po[r];
    }
#pragma unroll
    for (int q = 0; q < R1; ++q) mx = fmaxf(mx, mlv[q].x);
#pragma unroll
    for (int q = 0; q < R1; ++q) {
      if (q >= ns || mlv[q].x == -INFINITY) continue;
      const float f = exp2f(mlv[q].x - mx);
      L += f * mlv[q].y;
#pragma unroll
      for (int r = 0; r < CS / 4; ++r) {
        acc[4 * r + 0] += f * ov[q][r].x;
        acc[4 * r + 1] += f * ov[q][r].y;
        acc[4 * r + 2] += f * ov[q][r].z;
        acc[4 * r + 3] += f * ov[q][r].w;
      }
    }
  }
  for (int s0 = 0; s0 < (ns <= R1 ? 0 : ns); s0 += 4) {
    float mm[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) mm[q] = ml2[(size_t)(base + min(s0 + q, ns - 1)) * a.ucols + col].x;
#pragma unroll
    for (int q = 0; q < 4; ++q) mx = fmaxf(mx, mm[q]);
  }
  for (int s0 = 0; s0 < (ns <= R1 ? 0 : ns); s0 += 4) {
    float2 mlv[4];
    float4 ov[4][CS / 4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const size_t pi = (size_t)(base + min(s0 + q, ns - 1)) * a.ucols + col;
      mlv[q] = ml2[pi];
      const float4* po = reinterpret_cast<const float4*>(a.part_o + pi * a.hd + d0);
#pragma unroll
      for (int r = 0; r < CS / 4; ++r) ov[q][r] = po[r];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (s0 + q >= ns || mlv[q].x == -INFINITY) continue;
      const float f = exp2f(mlv[q].x - mx);
      L += f * mlv[q].y;
#pragma unroll
      for (int r = 0; r < CS / 4; ++r) {
        acc[4 * r + 0] += f * ov[q][r].x;
        acc[4 * r + 1] += f * ov[q][r].y;
        acc[4 * r + 2] += f * ov[q][r].z;
        acc[4 * r + 3] += f * ov[q][r].w;
      }
    }
  }
  const float invL = 1.0f / L;
  __shared__ float red[4];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < CS; ++i) {
    float v = acc[i] * invL;
    if (a.gate) {  // attn *= sigmoid(gate) (main.cpp:7697-7698, sigmoidf of :294)
      const float g = ifrd::h2f((uint16_t)(gw[i >> 1] >> (16 * (i & 1))));
      v *= 1.0f / (1.0f + expf(-g));
    }
    acc[i] = v;
    amax = fmaxf(amax, fabsf(v));
    if (own && a.attn_out) a.attn_out[(size_t)m * N + e0 + i] = v;
  }
  if (!own) amax = 0.0f;
  amax = ifrd::wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  const float mxa = fmaxf(1e-6f, fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
  const float sc = mxa / 127.0f;
  const float inv = 1.0f / sc;
  if (threadIdx.x == 0) a.qscale[m] = sc;
  // CS consecutive columns sit in one or two 16-byte A-tile lane chunks
  uint32_t w[CS / 4];
  int csum = 0;
#pragma unroll
  for (int i = 0; i < CS / 4; ++i) w[i] = 0u;
#pragma unroll
  for (int i = 0; i < CS; ++i) {
    const int c = ifrd::quant_half_away(acc[i], inv);
    w[i >> 2] |= (uint32_t)(c & 0xFF) << (8 * (i & 3));
    csum += c;
  }
  csum = group_sum_int<CS>(csum);
  if (!own) return;
  if constexpr (CS == 8) {
    *reinterpret_cast<uint2*>(a.q + atile_off(m, e0, N)) = make_uint2(w[0], w[1]);
  } else {
#pragma unroll
    for (int r = 0; r < CS / 16; ++r)
      *reinterpret_cast<uint4*>(a.q + atile_off(m, e0 + 16 * r, N)) =
          make_uint4(w[4 * r], w[4 * r + 1], w[4 * r + 2], w[4 * r + 3]);
  }
  if (threadIdx.x % (128 / CS) == 0) a.gsum[(size_t)m * (N / 128) + e0 / 128] = (float)csum;
}

}  // namespace

hipError_t launch_attention(const AttnArgs& a, const KVLayout& kv, hipStream_t st) {
  if (a.n_units <= 0) return hipSuccess;
  if (kv.hd != kHD || kv.page != kPage || a.nq % kv.nkv != 0 || (a.nq / kv.nkv) > 16 ||
      !a.units || !a.order || a.n_slots < a.n_units || !a.q || !a.part_o || !a.part_ml ||
      a.n_shared < 0 || a.n_shared % 4 != 0 || a.n_shared > a.n_slots || (kv.kv_int8 && a.n_shared))
    return hipErrorInvalidValue;
  const dim3 grid((a.n_slots + 3) / 4), block(256);
  if (a.col_tiles == 1) {
    if (kv.kv_int8) hipLaunchKernelGGL((attn_kernel<true, 1>), grid, block, 0, st, a, kv);
    else hipLaunchKernelGGL((attn_kernel<false, 1>), grid, block, 0, st, a, kv);
  } else if (a.col_tiles == 2) {
    if (kv.kv_int8) hipLaunchKernelGGL((attn_kernel<true, 2>), grid, block, 0, st, a, kv);
    else hipLaunchKernelGGL((attn_kernel<false, 2>), grid, block, 0, st, a, kv);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_combine(const CombineArgs& a, hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  const int N = a.nq * a.hd;
  if (N % 128 != 0 || N > 256 * 32 || a.hd != kHD || !a.q || !a.qscale || !a.gsum)
    return hipErrorInvalidValue;
  if (N <= 256 * 8) hipLaunchKernelGGL(combine_kernel<8>, dim3(a.M), dim3(256), 0, st, a);
  else if (N <= 256 * 16) hipLaunchKernelGGL(combine_kernel<16>, dim3(a.M), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(combine_kernel<32>, dim3(a.M), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace ifrk
