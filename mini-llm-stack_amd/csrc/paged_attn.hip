// Paged-attention decode (kernels/paged_attention.py:33-118): one query token per
// sequence attends to its keys/values scattered over fixed-size blocks of a shared
// pool, walked through the sequence's block table, with an online softmax. No copies
// of the context and no score vector longer than one block.
//
// Pools [num_blocks][H][block_size][D] (one (block, head) slab contiguous), strides
// (kv_sb, kv_sh, kv_st, 1) shared by K and V as in the reference; q and out
// [n_seqs][H][D] with strides (q_ss, q_sh, 1) / (o_ss, o_sh, 1).
//
// HBM-bound: every context key and value row is read once. Work unit: one wavefront
// per (sequence, head, context split). Lane l owns the 16-byte chunk `l % CPT` of
// token slot `l / CPT` (CPT = 16-byte chunks per row), so one load instruction
// covers 64 / CPT whole rows and each lane keeps only its EPC elements of q and of
// the output accumulator. A row's score is reduced over its CPT lanes with DPP moves
// (up to 16 lanes; wider rows add xor shuffles). Each lane runs its own online softmax (running max m, sum l,
// accumulator) over the tokens it sees; at the end the 64 / CPT token slots are
// merged pairwise (rescaling by exp(m - M)), then, when the context is split over
// several wavefronts, a second kernel merges the splits the same way from a
// workspace of (m, l, acc[D]) per split.
//
// Tokens at or past the context length score -inf (weight 0), so stale or poisoned
// cache slots in a partially filled block never leak in; a block id outside
// [0, num_blocks) is skipped (its tokens weigh 0) rather than dereferenced, and a
// context longer than the table row covers is cut at the row's end. A zero context
// gives a zero output, as in the reference.
#include <atomic>
#include <mutex>

#include "common.h"

namespace mls {

namespace {
typedef uint32_t kv16_t __attribute__((ext_vector_type(4)));  // 16 bytes of K or V
}  // namespace


namespace {

constexpr float NEG_INF = -__builtin_huge_valf();

// 16 bytes of T -> EPC floats
template <typename T>
__device__ __forceinline__ void load_chunk(const T* p, float* o) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  if constexpr (sizeof(T) == 4) {
    o[0] = __uint_as_float(v.x);
    o[1] = __uint_as_float(v.y);
    o[2] = __uint_as_float(v.z);
    o[3] = __uint_as_float(v.w);
  } else {
    const T* h = reinterpret_cast<const T*>(&v);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = to_f32(h[i]);
  }
}

// Merge two online-softmax states (m, l, acc) into the first.
template <int EPC>
__device__ __forceinline__ void merge_state(float& m, float& l, float* acc, float m2, float l2, const float* acc2) {
  const float M = fmaxf(m, m2);
  const float f1 = M == NEG_INF ? 0.0f : __expf(m - M);
  const float f2 = M == NEG_INF ? 0.0f : __expf(m2 - M);
  l = l * f1 + l2 * f2;
#pragma unroll
  for (int e = 0; e < EPC; ++e) acc[e] = acc[e] * f1 + acc2[e] * f2;
  m = M;
}

struct PagedArgs {
  const void* q;
  int64_t q_ss, q_sh;
  const void* kp;
  const void* vp;
  int64_t kv_sb, kv_sh, kv_st, num_blocks;
  const int32_t* bt;
  int64_t bt_ss, max_blocks;
  const int32_t* ctx;
  void* out;
  int64_t o_ss, o_sh;
  int n_seqs, H, D, BS;
  float scale;
  float* ws;  // splits > 1: [n_seqs][H][splits][D + 2] (acc[D], m, l)
  int splits;
};

template <typename QT, typename KT, int CPT>
__global__ __launch_bounds__(256) void paged_attn_kernel(const PagedArgs a) {
  constexpr int EPC = 16 / sizeof(KT);  // elements per 16-byte chunk
  constexpr int TPI = 64 / CPT;         // token slots per load instruction
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t items = (int64_t)a.n_seqs * a.H * a.splits;
  if (item >= items) return;
  // wave-uniform indices (readfirstlane), so table entries and lengths are scalar
  // loads, outside the vector-load counter that paces the K/V prefetch
  const int split = __builtin_amdgcn_readfirstlane((int)(item % a.splits));
  const int head = __builtin_amdgcn_readfirstlane((int)((item / a.splits) % a.H));
  const int seq = __builtin_amdgcn_readfirstlane((int)(item / ((int64_t)a.splits * a.H)));
  const int ts = lane / CPT, part = lane % CPT;

  float q[EPC];
  {
    const QT* qp = static_cast<const QT*>(a.q) + seq * a.q_ss + head * a.q_sh + part * EPC;
#pragma unroll
    for (int e = 0; e < EPC; ++e) q[e] = to_f32(qp[e]);
  }
  const int ctx = a.ctx[seq];
  const int nb = (int)min((int64_t)((max(ctx, 0) + a.BS - 1) / a.BS), a.max_blocks);  // never past the table row
  const int per = (nb + a.splits - 1) / a.splits;
  const int b0 = split * per, b1 = min(nb, b0 + per);

  float m = NEG_INF, l = 0.0f, acc[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) acc[e] = 0.0f;

  // A step is UNR load instructions of TPI tokens each (K and V chunks: 2 UNR 16-byte
  // loads per lane); a block of BS tokens takes spb steps. The chunks of step i + 1
  // are in flight while step i is scored, in two named register sets used
  // alternately (a register copy of a pending load would wait for it).
  constexpr int UNR = 4;
  const int spb = (a.BS + UNR * TPI - 1) / (UNR * TPI);
  const int total = a.num_blocks > 0 ? (b1 - b0) * spb : 0;
  const KT* kbase = static_cast<const KT*>(a.kp) + head * a.kv_sh + part * EPC;
  const KT* vbase = static_cast<const KT*>(a.vp) + head * a.kv_sh + part * EPC;
  const int32_t* table = a.bt + (int64_t)seq * a.bt_ss;
  auto issue = [&](int step, uint4 (&kr)[UNR], uint4 (&vr)[UNR], bool& ok) __attribute__((always_inline)) {
    const int b = b0 + step / spb, t0 = (step % spb) * UNR * TPI;
    const int blk = table[b];
    ok = blk >= 0 && blk < a.num_blocks;  // uniform over the wavefront
    // unconditional loads (a branch around them would make the compiler wait for
    // each): an invalid block reads block 0, a slot past the block end reads the
    // block's last token; score() gives both weight 0
    const int64_t boff = ok ? (int64_t)blk * a.kv_sb : 0;
    // non-temporal: every cached K / V byte is read once per call (the 64 x 32 x 2048 bench
    // shape: 368 -> 330 us against the default policy)
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int t = min(t0 + u * TPI + ts, a.BS - 1);
      kr[u] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const kv16_t*>(kbase + boff + t * a.kv_st)));
      vr[u] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const kv16_t*>(vbase + boff + t * a.kv_st)));
    }
  };
  auto score = [&](int step, const uint4 (&kr)[UNR], const uint4 (&vr)[UNR], bool ok) __attribute__((always_inline)) {
    const int b = b0 + step / spb, t0 = (step % spb) * UNR * TPI;
    float sc[UNR];
    float mx = m;
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      float kv[EPC];
      load_chunk(reinterpret_cast<const KT*>(&kr[u]), kv);
      float s = 0.0f;
#pragma unroll
      for (int e = 0; e < EPC; ++e) s = fmaf(q[e], kv[e], s);
      s = lane_group_sum<CPT>(s);
      const int t = t0 + u * TPI + ts;
      sc[u] = (ok && t < a.BS && b * a.BS + t < ctx) ? s * a.scale : NEG_INF;
      mx = fmaxf(mx, sc[u]);
    }
    // (no early exit: a branch here would make the compiler wait on the prefetch;
    // with nothing valid so far and in this step, every weight below is 0)
    const float al = m == NEG_INF ? 0.0f : __expf(m - mx);
    l *= al;
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc[e] *= al;
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const float p = sc[u] == NEG_INF ? 0.0f : __expf(sc[u] - mx);
      float vv[EPC];
      load_chunk(reinterpret_cast<const KT*>(&vr[u]), vv);
      l += p;
#pragma unroll
      for (int e = 0; e < EPC; ++e) acc[e] = fmaf(p, vv[e], acc[e]);
    }
    m = mx;
  };
  uint4 ka[UNR], va[UNR], kb[UNR], vb[UNR];
  bool oka = false, okb = false;
  // branch-free pairs of steps: the step indices are clamped (a repeated last step is
  // loaded again and scored with weight 0)
  if (total > 0) issue(0, ka, va, oka);
  for (int step = 0; step < total; step += 2) {
    issue(min(step + 1, total - 1), kb, vb, okb);
    score(step, ka, va, oka);
    issue(min(step + 2, total - 1), ka, va, oka);
    score(step + 1, kb, vb, okb && step + 1 < total);
  }
  // merge the token slots that share this lane's chunk (lanes part, part + CPT, ...)
#pragma unroll
  for (int o = CPT; o < 64; o <<= 1) {
    const float m2 = __shfl_xor(m, o), l2 = __shfl_xor(l, o);
    float acc2[EPC];
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc2[e] = __shfl_xor(acc[e], o);
    merge_state<EPC>(m, l, acc, m2, l2, acc2);
  }
  if (ts != 0) return;
  if (a.splits == 1) {
    const float inv = l == 0.0f ? 1.0f : 1.0f / l;
    QT* op = static_cast<QT*>(a.out) + seq * a.o_ss + head * a.o_sh + part * EPC;
#pragma unroll
    for (int e = 0; e < EPC; ++e) op[e] = from_f32<QT>(acc[e] * inv);
  } else {
    float* w = a.ws + (((int64_t)seq * a.H + head) * a.splits + split) * (a.D + 2);
#pragma unroll
    for (int e = 0; e < EPC; ++e) w[part * EPC + e] = acc[e];
    if (part == 0) {
      w[a.D] = m;
      w[a.D + 1] = l;
    }
  }
}

// Any D and stride: one wavefront per (sequence, head, split), lane d owns elements
// d, d + 64, d + 128, d + 192 (D <= 256); one token at a time, wave-wide dot product.
template <typename QT, typename KT>
__global__ __launch_bounds__(256) void paged_attn_generic_kernel(const PagedArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)a.n_seqs * a.H * a.splits) return;
  const int split = (int)(item % a.splits);
  const int head = (int)((item / a.splits) % a.H);
  const int seq = (int)(item / ((int64_t)a.splits * a.H));
  float q[4], acc[4] = {0.f, 0.f, 0.f, 0.f};
  const QT* qp = static_cast<const QT*>(a.q) + seq * a.q_ss + head * a.q_sh;
#pragma unroll
  for (int i = 0; i < 4; ++i) q[i] = lane + 64 * i < a.D ? to_f32(qp[lane + 64 * i]) : 0.0f;
  const int ctx = a.ctx[seq];
  const int nb = (int)min((int64_t)((max(ctx, 0) + a.BS - 1) / a.BS), a.max_blocks);  // never past the table row
  const int per = (nb + a.splits - 1) / a.splits;
  const int b0 = split * per, b1 = min(nb, b0 + per);
  float m = NEG_INF, l = 0.0f;
  const int32_t* table = a.bt + (int64_t)seq * a.bt_ss;
  for (int b = b0; b < b1; ++b) {
    const int blk = table[b];
    if (blk < 0 || blk >= a.num_blocks) continue;
    for (int t = 0; t < a.BS && b * a.BS + t < ctx; ++t) {
      const int64_t off = (int64_t)blk * a.kv_sb + head * a.kv_sh + t * a.kv_st;
      const KT* kr = static_cast<const KT*>(a.kp) + off;
      const KT* vr = static_cast<const KT*>(a.vp) + off;
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (lane + 64 * i < a.D) s = fmaf(q[i], to_f32(kr[lane + 64 * i]), s);
      s = wave_sum(s) * a.scale;
      const float mn = fmaxf(m, s);
      const float al = m == NEG_INF ? 0.0f : __expf(m - mn);
      const float p = __expf(s - mn);
      l = l * al + p;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[i] = fmaf(p, lane + 64 * i < a.D ? to_f32(vr[lane + 64 * i]) : 0.0f, acc[i] * al);
      m = mn;
    }
  }
  if (a.splits == 1) {
    const float inv = l == 0.0f ? 1.0f : 1.0f / l;
    QT* op = static_cast<QT*>(a.out) + seq * a.o_ss + head * a.o_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (lane + 64 * i < a.D) op[lane + 64 * i] = from_f32<QT>(acc[i] * inv);
  } else {
    float* w = a.ws + (((int64_t)seq * a.H + head) * a.splits + split) * (a.D + 2);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (lane + 64 * i < a.D) w[lane + 64 * i] = acc[i];
    if (lane == 0) {
      w[a.D] = m;
      w[a.D + 1] = l;
    }
  }
}

// Merge the splits of one (sequence, head): one wavefront, lanes over D.
template <typename QT>
__global__ __launch_bounds__(256) void paged_attn_merge_kernel(const PagedArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)a.n_seqs * a.H) return;
  const int head = (int)(item % a.H), seq = (int)(item / a.H);
  const float* w = a.ws + item * a.splits * (a.D + 2);
  float M = NEG_INF;
  for (int s = 0; s < a.splits; ++s) M = fmaxf(M, w[s * (a.D + 2) + a.D]);
  float L = 0.0f;
  for (int s = 0; s < a.splits; ++s) {
    const float ms = w[s * (a.D + 2) + a.D];
    L += M == NEG_INF ? 0.0f : w[s * (a.D + 2) + a.D + 1] * __expf(ms - M);
  }
  const float inv = L == 0.0f ? 1.0f : 1.0f / L;
  QT* op = static_cast<QT*>(a.out) + seq * a.o_ss + head * a.o_sh;
  for (int d = lane; d < a.D; d += 64) {
    float acc = 0.0f;
    for (int s = 0; s < a.splits; ++s) {
      const float ms = w[s * (a.D + 2) + a.D];
      if (M != NEG_INF) acc = fmaf(w[s * (a.D + 2) + d], __expf(ms - M), acc);
    }
    op[d] = from_f32<QT>(acc * inv);
  }
}

// Context splits: enough wavefronts to cover the GPU several times over when there are
// few (sequence, head) pairs, each split at least 8 blocks of the table.
int choose_splits(int64_t n_seqs, int64_t H, int64_t max_blocks) {
  const int64_t items = n_seqs * H;
  if (items <= 0) return 1;
  int64_t s = cdiv(4096, items);
  const int64_t cap = cdiv(max_blocks, 8);
  s = s < cap ? s : cap;
  s = s > 1 ? s : 1;
  return (int)(s < 64 ? s : 64);
}

template <typename QT, typename KT>
int launch_paged(const PagedArgs& a, bool fast, int cpt, hipStream_t st) {
  const int64_t items = (int64_t)a.n_seqs * a.H * a.splits;
  const dim3 grid((unsigned)cdiv(items, 4)), block(256);
  if (fast) {
    switch (cpt) {
      case 1: hipLaunchKernelGGL((paged_attn_kernel<QT, KT, 1>), grid, block, 0, st, a); break;
      case 2: hipLaunchKernelGGL((paged_attn_kernel<QT, KT, 2>), grid, block, 0, st, a); break;
      case 4: hipLaunchKernelGGL((paged_attn_kernel<QT, KT, 4>), grid, block, 0, st, a); break;
      case 8: hipLaunchKernelGGL((paged_attn_kernel<QT, KT, 8>), grid, block, 0, st, a); break;
      case 16: hipLaunchKernelGGL((paged_attn_kernel<QT, KT, 16>), grid, block, 0, st, a); break;
      case 32: hipLaunchKernelGGL((paged_attn_kernel<QT, KT, 32>), grid, block, 0, st, a); break;
      default: hipLaunchKernelGGL((paged_attn_kernel<QT, KT, 64>), grid, block, 0, st, a); break;
    }
  } else {
    hipLaunchKernelGGL((paged_attn_generic_kernel<QT, KT>), grid, block, 0, st, a);
  }
  int rc = check_launch("mls_paged_attention_decode");
  if (rc != MLS_OK || a.splits == 1) return rc;
  hipLaunchKernelGGL((paged_attn_merge_kernel<QT>), dim3((unsigned)cdiv((int64_t)a.n_seqs * a.H, 4)), block, 0,
                     st, a);
  return check_launch("mls_paged_attention_decode(merge)");
}

template <typename QT>
int launch_paged_kv(const PagedArgs& a, int kv_dt, bool fast, int cpt, hipStream_t st) {
  if (kv_dt == MLS_F32) return launch_paged<QT, float>(a, fast, cpt, st);
  if (kv_dt == MLS_F16) return launch_paged<QT, _Float16>(a, fast, cpt, st);
  return launch_paged<QT, __bf16>(a, fast, cpt, st);
}

}  // namespace

}  // namespace mls

using namespace mls;

extern "C" int64_t mls_paged_attention_workspace(int64_t n_seqs, int64_t H, int64_t D, int64_t max_blocks) {
  if (n_seqs <= 0 || H <= 0 || D <= 0 || max_blocks <= 0) return 0;
  const int s = choose_splits(n_seqs, H, max_blocks);
  return s > 1 ? n_seqs * H * s * (D + 2) : 0;
}

namespace {

// Validates a decode call and fills `a` (workspace left null). *done: nothing to launch
// (an empty batch); *need: workspace floats the split merge needs (0: no split).
int paged_prepare(const char* fn, const void* q, int q_dt, int64_t q_ss, int64_t q_sh, const void* k_pool,
                  const void* v_pool, int kv_dt, int64_t kv_sb, int64_t kv_sh, int64_t kv_st, int64_t num_blocks,
                  const int32_t* block_tables, int64_t bt_ss, int64_t max_blocks, const int32_t* context_lens,
                  void* out, int64_t o_ss, int64_t o_sh, int64_t n_seqs, int64_t H, int64_t D, int64_t block_size,
                  float scale, PagedArgs& a, int64_t& need, bool& fast, int& cpt, bool& done) {
  done = false;
  if (n_seqs < 0 || H < 0 || D < 0 || block_size < 1 || max_blocks < 0 || num_blocks < 0)
    return fail(MLS_ERR_ARG, "%s: bad sizes n_seqs=%lld H=%lld D=%lld block_size=%lld", fn, (long long)n_seqs,
                (long long)H, (long long)D, (long long)block_size);
  if (!is_float_dt(q_dt) || !is_float_dt(kv_dt)) return fail(MLS_ERR_ARG, "%s: bad dtype", fn);
  if (n_seqs == 0 || H == 0 || D == 0) {
    done = true;
    return MLS_OK;
  }
  if (!q || !k_pool || !v_pool || !context_lens || !out || (max_blocks > 0 && !block_tables))
    return fail(MLS_ERR_ARG, "%s: null pointer", fn);
  if (q_sh < D || q_ss < H * D || o_sh < D || o_ss < H * D || kv_st < D || kv_sh < kv_st * block_size ||
      kv_sb < kv_sh * H || bt_ss < max_blocks)
    return fail(MLS_ERR_ARG, "%s: bad strides", fn);
  if (D > 256 && D * dt_size(kv_dt) > 1024)
    return fail(MLS_ERR_UNSUPPORTED, "%s: head dim %lld too large", fn, (long long)D);
  if (n_seqs * H > 0x3FFFFFFF || block_size > 0x3FFFFFFF)
    return fail(MLS_ERR_UNSUPPORTED, "%s: too large", fn);
  const int splits = choose_splits(n_seqs, H, max_blocks);
  need = splits > 1 ? n_seqs * H * splits * (D + 2) : 0;
  const int esz = dt_size(kv_dt);
  const int64_t row = D * esz;
  cpt = (int)(row / 16);
  fast = row % 16 == 0 && cpt >= 1 && cpt <= 64 && (cpt & (cpt - 1)) == 0 && (kv_st * esz) % 16 == 0 &&
         (kv_sh * esz) % 16 == 0 && (kv_sb * esz) % 16 == 0 && aligned(k_pool, 16) && aligned(v_pool, 16);
  if (!fast && D > 256) return fail(MLS_ERR_UNSUPPORTED, "%s: head dim %lld needs 16-byte rows", fn, (long long)D);
  a = PagedArgs{q, q_ss, q_sh, k_pool, v_pool, kv_sb, kv_sh, kv_st, num_blocks, block_tables, bt_ss,
                max_blocks, context_lens, out, o_ss, o_sh, (int)n_seqs, (int)H, (int)D, (int)block_size,
                scale, nullptr, splits};
  return MLS_OK;
}

int paged_launch(const PagedArgs& a, int q_dt, int kv_dt, bool fast, int cpt, hipStream_t st) {
  if (q_dt == MLS_F32) return launch_paged_kv<float>(a, kv_dt, fast, cpt, st);
  if (q_dt == MLS_F16) return launch_paged_kv<_Float16>(a, kv_dt, fast, cpt, st);
  return launch_paged_kv<__bf16>(a, kv_dt, fast, cpt, st);
}

}  // namespace

extern "C" int mls_paged_attention_decode(const void* q, int q_dt, int64_t q_ss, int64_t q_sh,
                                          const void* k_pool, const void* v_pool, int kv_dt, int64_t kv_sb,
                                          int64_t kv_sh, int64_t kv_st, int64_t num_blocks,
                                          const int32_t* block_tables, int64_t bt_ss, int64_t max_blocks,
                                          const int32_t* context_lens, void* out, int64_t o_ss, int64_t o_sh,
                                          int64_t n_seqs, int64_t H, int64_t D, int64_t block_size, float scale,
                                          float* workspace, int64_t workspace_floats, mls_stream_t stream) {
  const char* fn = "mls_paged_attention_decode";
  PagedArgs a{};
  int64_t need = 0;
  bool fast = false, done = false;
  int cpt = 0;
  int rc = paged_prepare(fn, q, q_dt, q_ss, q_sh, k_pool, v_pool, kv_dt, kv_sb, kv_sh, kv_st, num_blocks,
                         block_tables, bt_ss, max_blocks, context_lens, out, o_ss, o_sh, n_seqs, H, D, block_size,
                         scale, a, need, fast, cpt, done);
  if (rc != MLS_OK || done) return rc;
  if (need > 0 && (!workspace || workspace_floats < need))
    return fail(MLS_ERR_ARG, "%s: workspace of %lld floats needed (mls_paged_attention_workspace)", fn,
                (long long)need);
  a.ws = workspace;
  return paged_launch(a, q_dt, kv_dt, fast, cpt, (hipStream_t)stream);
}

// ---------------------------------------------------------------- allocation-free variant
//
// The split partials (acc[D], m, l per split) live in `scratch`, a device array of
// MLS_PAGED_SCRATCH_FLOATS floats (8 MiB) that every GPU this library runs on holds
// until the process ends. Host code never passes the array's name to a kernel (in host
// code it names a host-side stand-in): the device address comes from
// hipGetSymbolAddress, taken once per device with that device current, and is kept in
// scratch_dev[]. No entry of the workspace needs to start at zero: every split writes
// its whole (acc, m, l) record, empty splits included, before the merge kernel reads
// it. All calls on one GPU share its array, so calls that overlap on one GPU (two
// streams, or two host threads) race on it.

static __device__ __align__(256) float scratch[MLS_PAGED_SCRATCH_FLOATS];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<float*> scratch_dev[kMaxDevices];
std::mutex scratch_mu;

// The device address of `scratch` on the device that owns stream `st`.
int scratch_for(hipStream_t st, float** ptr, const char* fn) {
  int dev = -1;
  hipError_t e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MLS_ERR_HIP, "%s: stream device: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MLS_ERR_UNSUPPORTED, "%s: device %d", fn, dev);
  float* p = scratch_dev[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(scratch_mu);
    p = scratch_dev[dev].load(std::memory_order_relaxed);
    if (!p) {
      int cur = -1;
      e = hipGetDevice(&cur);
      if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
      void* sym = nullptr;
      if (e == hipSuccess) e = hipGetSymbolAddress(&sym, HIP_SYMBOL(scratch));
      if (cur >= 0 && cur != dev) {
        const hipError_t e2 = hipSetDevice(cur);
        if (e == hipSuccess) e = e2;
      }
      if (e != hipSuccess || !sym)
        return fail(MLS_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", fn, hipGetErrorString(e));
      p = static_cast<float*>(sym);
      scratch_dev[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return MLS_OK;
}

}  // namespace

extern "C" int mls_paged_attention_decode_noalloc(const void* q, int q_dt, int64_t q_ss, int64_t q_sh,
                                                  const void* k_pool, const void* v_pool, int kv_dt, int64_t kv_sb,
                                                  int64_t kv_sh, int64_t kv_st, int64_t num_blocks,
                                                  const int32_t* block_tables, int64_t bt_ss, int64_t max_blocks,
                                                  const int32_t* context_lens, void* out, int64_t o_ss,
                                                  int64_t o_sh, int64_t n_seqs, int64_t H, int64_t D,
                                                  int64_t block_size, float scale, mls_stream_t stream) {
  const char* fn = "mls_paged_attention_decode_noalloc";
  PagedArgs a{};
  int64_t need = 0;
  bool fast = false, done = false;
  int cpt = 0;
  int rc = paged_prepare(fn, q, q_dt, q_ss, q_sh, k_pool, v_pool, kv_dt, kv_sb, kv_sh, kv_st, num_blocks,
                         block_tables, bt_ss, max_blocks, context_lens, out, o_ss, o_sh, n_seqs, H, D, block_size,
                         scale, a, need, fast, cpt, done);
  if (rc != MLS_OK || done) return rc;
  if (need > MLS_PAGED_SCRATCH_FLOATS)
    return fail(MLS_ERR_ARG,
                "%s: the context split of this call needs %lld workspace floats, above the static scratch of %lld; "
                "use mls_paged_attention_decode with a caller workspace",
                fn, (long long)need, (long long)MLS_PAGED_SCRATCH_FLOATS);
  if (need > 0) {
    rc = scratch_for((hipStream_t)stream, &a.ws, fn);
    if (rc != MLS_OK) return rc;
  }
  return paged_launch(a, q_dt, kv_dt, fast, cpt, (hipStream_t)stream);
}
