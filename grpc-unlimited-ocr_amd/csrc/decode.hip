// decode.hip: the key/value-cache ops of one decode step for gfx950, with
// every length-dependent value read from the device StepState so that a
// captured step replays for every token (the reference's append_step and
// attend_step, src/backend/cuda/decode_ops.h:28-47, decode_ops.cu:49-52,
// 112-195).
//
// append_step: cache[pos, :] = row, one 16-byte chunk per thread.
//
// attend_step: out[h] = softmax(q_h . K_h^T * scale + mask) V_h over the keys
// 0..pos of a cache [capacity, heads * hd], one query row. Split-K in two
// launches of fixed shape:
//   partial  grid heads x splits, 4 waves each. A split owns a contiguous
//            run of keys (its length follows pos). Inside a wave, G lanes
//            share a key (each holds VW * VPL elements of the head), so
//            64 / G keys are scored at once; a lane group walks its keys U
//            at a time with an online softmax (running max m, total l and
//            weighted sum of value rows), so no score array is kept. Masked
//            keys (-inf) are neither scored nor read. The 4 * 64 / G lane
//            groups then fold through LDS into one (m, l, acc[hd]) record
//            per split.
//   merge    one workgroup per (head, 64 elements of the head) folds the
//            splits' records and writes out = acc / l (zeros when every key
//            is masked).
// Scores are s = (q . k) * scale + mask (two roundings, as the reference's
// CPU attention forms them, src/backend/reference/ops.cpp:219-251); every
// exponential is 2^((s - m) log2 e) on v_exp_f32.

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr int64_t kMaxHeadDim = 256;
constexpr int kMaxSplits = 128;
constexpr int kMaskTile = 2048;
// The live-key segments a routed step attends to (the key segments of
// uocr_rocm.h):
// a header of 4 words and up to kMaxKeySegments segments of 4 words.
constexpr int kMaxKeySegments = UOCR_ROCM_MAX_KEY_SEGMENTS;
constexpr int kSegWords = 4 * (1 + kMaxKeySegments);

// ---- append ---------------------------------------------------------------------

// TC is the cache's element type: float, or uint16_t for a bf16 cache (the
// fp32 row rounded to nearest even on the way in).
template <class TC, int VW>
__global__ __launch_bounds__(kBlock) void append_k(TC* __restrict__ cache, const float* __restrict__ row,
                                                   int64_t width, const uocr_rocm_step_state* __restrict__ state,
                                                   int64_t capacity) {
  const int64_t pos = state->pos;
  if (pos < 0 || (capacity >= 0 && pos >= capacity)) return;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (c * VW >= width) return;
  Chunk<float, VW> v;
  v.load(row + c * VW);
  float f[VW];
  v.widen(f);
  Chunk<TC, VW> o;
  o.narrow(f);
  o.store(cache + pos * width + c * VW);
}

// ---- attention ------------------------------------------------------------------

// Sum over aligned groups of G lanes; every lane of a group ends with the
// same bits (each step adds the same two operands in either lane).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += dpp_f32<0xB1>(v);   // lane ^ 1
  if constexpr (G >= 4) v += dpp_f32<0x4E>(v);   // lane ^ 2
  if constexpr (G >= 8) v += dpp_f32<0x141>(v);  // the two quads of 8 lanes
  if constexpr (G >= 16) v += dpp_f32<0x140>(v); // the two halves of 16 lanes
  if constexpr (G >= 32) {
    // ds_swizzle bit mode: and 0x1f, xor 0x10 -> lane ^ 16 within 32 lanes.
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  }
  if constexpr (G >= 64) v += __shfl_xor(v, 32);
  return v;
}

struct AttendArgs {
  const float* q;
  const void* k;  // caches of element type TC (float or bf16 bits)
  const void* v;
  const float* mask;
  float* part;  // [heads, splits, hd + 2]: m, l, acc[hd]
  const uocr_rocm_step_state* state;
  int64_t width;
  int64_t capacity;
  float scale;
  int hd;
  int splits;
  // With rope and append (kRope): the step's new K and V rows [width], the
  // caches to append them to, and the rope tables.
  const float* k_row;
  const float* v_row;
  void* k_out;
  void* v_out;
  const float* inv_tok;
  const float* inv_page;
  int64_t page_mod;
  int n_tok;
  // With segments (kSegs): the live keys as segments, in place of the mask.
  const int* segs;
};


// The K and V chunks of U keys of one lane group, with each key's mask value
// (-inf for a key that is masked or past the end: such a key is not read).
template <class TC, int VW, int VPL, int U>
struct KeyBatch {
  Chunk<TC, VW> k[U][VPL];
  Chunk<TC, VW> v[U][VPL];
  float mk[U];
  bool is_new[U];  // the step's own key (kRope): its K and V come from LDS
};

// One lane group's running softmax state over its keys.
template <int VW, int VPL>
struct Running {
  float m = -INFINITY;
  float l = 0.0f;
  float acc[VPL][VW];
};

__device__ __forceinline__ float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// kSegs: the split owns a run of the live keys (the segments' keys in
// order) instead of a run of positions; each tile stages its keys' positions
// and biases in LDS, and split 0 appends the step's key and value (a
// workgroup that meets key pos takes it from its own rotated copy).
template <class TC, int VW, int G, int VPL, int U, bool kRope, bool kEarly, bool kSegs = false>
__global__ __launch_bounds__(kBlock) void attend_partial(const AttendArgs a) {
  static_assert(kRope || !kEarly, "the early first batch is the rope kernel's (and only without a mask)");
  static_assert(!(kSegs && kEarly), "the early first batch needs no mask and no segments");
  constexpr bool kBf16 = sizeof(TC) == 2;
  const TC* kc = static_cast<const TC*>(a.k);
  const TC* vc = static_cast<const TC*>(a.v);
  // A key that is masked or past the end reads the query row instead (valid,
  // cached, never used); for a bf16 cache its bytes are read as bf16 bits.
  const TC* dead = reinterpret_cast<const TC*>(a.q);
  constexpr int kSlotsPerWave = kWave / G;
  constexpr int kSlots = kWavesPerBlock * kSlotsPerWave;
  constexpr int kPerLane = VW * VPL;
  constexpr int64_t kStride = static_cast<int64_t>(kSlots) * U;  // keys per lane-group batch
  static_assert(kMaskTile % kStride == 0, "mask tiles hold whole batches");
  __shared__ float s_mask[kMaskTile];
  __shared__ int s_key[kSegs ? kMaskTile : 1];
  __shared__ int s_seg[kSegs ? kSegWords : 1];
  __shared__ float s_m[kSlots];
  __shared__ float s_l[kSlots];
  __shared__ float s_acc[kSlots * G * kPerLane];
  __shared__ float s_new[kRope ? 3 : 1][kRope ? kMaxHeadDim : 1];  // rotated q, rotated k, v of this head

  // Split-major: the heads' workgroups of one key range are dispatched
  // together and read the same cache rows.
  const int heads = static_cast<int>(a.width / a.hd);
  const int h = blockIdx.x % heads, split = blockIdx.x / heads;
  const int lane = threadIdx.x & (kWave - 1);
  const int slot = (threadIdx.x / kWave) * kSlotsPerWave + lane / G;
  const int gl = lane % G;
  const int64_t pos = a.state->pos;
  int64_t keys = pos + 1;
  keys = keys < 0 ? 0 : (keys > a.capacity ? a.capacity : keys);
  if constexpr (kSegs) {
    for (int t = static_cast<int>(threadIdx.x); t < kSegWords; t += kBlock) s_seg[t] = a.segs[t];
    __syncthreads();
    const int64_t live = s_seg[1];
    keys = pos < 0 || pos >= a.capacity || live < 0 ? 0 : live;
  }
  const int64_t chunk = (keys + a.splits - 1) / a.splits;
  const int64_t first = split * chunk;
  const int64_t last = first + chunk < keys ? first + chunk : keys;
  const int nvec = a.hd / VW;
  const int64_t head_off = static_cast<int64_t>(h) * a.hd;

  // This lane's chunks of the head: c = gl + G i; lanes past the head (when
  // nvec is not a power of two) address the head's last chunk and their
  // values are dropped.
  int64_t col[VPL];
  bool in_head[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = gl + G * i;
    in_head[i] = c < nvec;
    col[i] = head_off + static_cast<int64_t>(in_head[i] ? c : nvec - 1) * VW;
  }

  // Loads are issued unconditionally: a key that is masked or past the end
  // reads the query row instead (cached; its score is -inf and its value is
  // replaced by 0), so the loop has no branch around a load and the next
  // batch's loads stay in flight while the current batch is scored.
  auto issue = [&](KeyBatch<TC, VW, VPL, U>& b, int64_t jb, int64_t t0, int64_t t1) {
    int64_t kp[U];  // the keys' positions
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = jb + static_cast<int64_t>(kSlots) * u;
      const bool in = j < t1;
      if constexpr (kSegs) {
        kp[u] = in ? s_key[j - t0] : 0;
        b.mk[u] = in ? s_mask[j - t0] : -INFINITY;
      } else {
        kp[u] = j;
        b.mk[u] = in ? (a.mask != nullptr ? s_mask[j - t0] : 0.0f) : -INFINITY;
      }
      b.is_new[u] = kRope && in && kp[u] == pos;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = b.mk[u] != -INFINITY && !b.is_new[u];
#pragma unroll
      for (int i = 0; i < VPL; ++i) b.k[u][i].load(live ? kc + kp[u] * a.width + col[i] : dead + col[i]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = b.mk[u] != -INFINITY && !b.is_new[u];
#pragma unroll
      for (int i = 0; i < VPL; ++i) b.v[u][i].load(live ? vc + kp[u] * a.width + col[i] : dead + col[i]);
    }
  };

  KeyBatch<TC, VW, VPL, U> A, B;

  if constexpr (kRope) {
    // rope on this head's q and new k, with rope.hip's arithmetic: angle =
    // float(tok) inv_tok[p] (or float(page mod page_mod) inv_page[p - n_tok]),
    // device sincosf, a c - b s / b c + a s without contraction. Thread p
    // takes pair p and element p of v (hd <= kBlock: one of each at most).
    // The row loads are unconditional (indices clamped into the head) and
    // issued first: without a mask (kEarly) the first key batch follows
    // them at once, and as a wave's loads complete in order, the rope
    // arithmetic then waits for the rows only while the batch is in flight.
    static_assert(kMaxHeadDim <= kBlock, "one rope pair and one v element per thread");
    const int half = a.hd / 2;
    const int p = threadIdx.x;
    const int pc = p < half ? p : half - 1, tc = p < a.hd ? p : a.hd - 1;
    const float qa = a.q[head_off + pc], qb = a.q[head_off + pc + half];
    const float ka = a.k_row[head_off + pc], kb = a.k_row[head_off + pc + half];
    const float inv = *(pc < a.n_tok ? a.inv_tok + pc : a.inv_page + (pc - a.n_tok));
    const float vr = a.v_row[head_off + tc];
    if constexpr (kEarly) issue(A, first + slot, first, last);
    int64_t pg = a.state->page;
    if (a.page_mod > 0) pg = ((pg % a.page_mod) + a.page_mod) % a.page_mod;
    const float ft = static_cast<float>(a.state->tok), fp = static_cast<float>(pg);
    if (p < half) {
      const float angle = (p < a.n_tok ? ft : fp) * inv;
      float sn, cs;
      sincosf(angle, &sn, &cs);
      {
#pragma clang fp contract(off)
        s_new[0][p] = qa * cs - qb * sn;
        s_new[0][p + half] = qb * cs + qa * sn;
        s_new[1][p] = ka * cs - kb * sn;
        s_new[1][p + half] = kb * cs + ka * sn;
      }
      if constexpr (kBf16) {  // the key as the bf16 cache will hold it
        s_new[1][p] = round_bf16(s_new[1][p]);
        s_new[1][p + half] = round_bf16(s_new[1][p + half]);
      }
    }
    if (p < a.hd) s_new[2][p] = kBf16 ? round_bf16(vr) : vr;
    __syncthreads();
    // The split that holds key pos appends the head's rotated k and its v
    // (with segments: split 0, whether or not key pos is live).
    const bool appends = kSegs ? split == 0 && pos >= 0 && pos < a.capacity : pos >= first && pos < last;
    if (appends) {
      for (int t = threadIdx.x; t < a.hd; t += kBlock) {
        Chunk<TC, 1> kk, vv;
        kk.narrow({s_new[1][t]});
        vv.narrow({s_new[2][t]});
        kk.store(static_cast<TC*>(a.k_out) + pos * a.width + head_off + t);
        vv.store(static_cast<TC*>(a.v_out) + pos * a.width + head_off + t);
      }
    }
  }

  float qv[VPL][VW];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
#pragma unroll
    for (int e = 0; e < VW; ++e) {
      if constexpr (kRope) {
        qv[i][e] = in_head[i] ? s_new[0][col[i] - head_off + e] : 0.0f;
      } else {
        qv[i][e] = in_head[i] ? a.q[col[i] + e] : 0.0f;
      }
    }
  }

  Running<VW, VPL> run;
#pragma unroll
  for (int i = 0; i < VPL; ++i)
#pragma unroll
    for (int e = 0; e < VW; ++e) run.acc[i][e] = 0.0f;

  auto consume = [&](const KeyBatch<TC, VW, VPL, U>& b) {
    float s[U];
    float peak = run.m;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float d = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float kv[VW];
        b.k[u][i].widen(kv);
        if constexpr (kRope) {
          if (b.is_new[u]) {
#pragma unroll
            for (int e = 0; e < VW; ++e) kv[e] = s_new[1][col[i] - head_off + e];
          }
        }
#pragma unroll
        for (int e = 0; e < VW; ++e) d = fmaf(qv[i][e], in_head[i] ? kv[e] : 0.0f, d);
      }
      d = group_sum<G>(d);
      {
#pragma clang fp contract(off)
        s[u] = b.mk[u] != -INFINITY ? d * a.scale + b.mk[u] : -INFINITY;
      }
      peak = fmaxf(peak, s[u]);
    }
    if (peak == -INFINITY) return;  // uniform over the lane group
    const float alpha = exp_shift(run.m, peak);
    run.l *= alpha;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int e = 0; e < VW; ++e) run.acc[i][e] *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float p = exp_shift(s[u], peak);
      run.l += p;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float vv[VW];
        b.v[u][i].widen(vv);
        if constexpr (kRope) {
          if (b.is_new[u]) {
#pragma unroll
            for (int e = 0; e < VW; ++e) vv[e] = s_new[2][col[i] - head_off + e];
          }
        }
        // A dead key (masked or past the end) holds filler bits, which need
        // not be finite (bf16 halves of the query row can be NaN): its value
        // enters as 0, never as 0 * filler.
        const bool use = in_head[i] && b.mk[u] != -INFINITY;
#pragma unroll
        for (int e = 0; e < VW; ++e) run.acc[i][e] = fmaf(p, use ? vv[e] : 0.0f, run.acc[i][e]);
      }
    }
    run.m = peak;
  };

  // Key tiles: the mask of a tile is staged in LDS by the whole workgroup
  // (one coalesced load per thread per 256 keys); without a mask the split
  // is one tile.
  const int64_t tile = kSegs || a.mask != nullptr ? kMaskTile : (last > first ? last - first : 1);
  for (int64_t t0 = first; t0 < last; t0 += tile) {
    const int64_t t1 = t0 + tile < last ? t0 + tile : last;
    if constexpr (kSegs) {
      // live key j of this tile: the segment holding it (segments in key
      // order), its position (at most pos) and its bias
      __syncthreads();  // the previous tile's readers are done
      const int nseg = s_seg[0] < kMaxKeySegments ? s_seg[0] : kMaxKeySegments;
      for (int64_t j = t0 + threadIdx.x; j < t1; j += kBlock) {
        int64_t cum = 0, key = 0;
        float bias = -INFINITY;
        for (int g = 0; g < nseg; ++g) {
          const int64_t len = s_seg[4 * (1 + g) + 1];
          if (j < cum + len) {
            key = s_seg[4 * (1 + g)] + (j - cum);
            bias = __int_as_float(s_seg[4 * (1 + g) + 2]);
            break;
          }
          cum += len;
        }
        s_key[j - t0] = static_cast<int>(key < 0 ? 0 : (key > pos ? pos : key));
        s_mask[j - t0] = bias;
      }
      __syncthreads();
    } else if (a.mask != nullptr) {
      constexpr int kPer = kMaskTile / kBlock;
      float mv[kPer];
#pragma unroll
      for (int r = 0; r < kPer; ++r) {
        const int64_t j = t0 + threadIdx.x + static_cast<int64_t>(r) * kBlock;
        mv[r] = a.mask[j < t1 ? j : t1 - 1];
      }
      __syncthreads();  // the previous tile's readers are done
#pragma unroll
      for (int r = 0; r < kPer; ++r) s_mask[threadIdx.x + r * kBlock] = mv[r];
      __syncthreads();
    }
    const int64_t base = t0 + slot;
    const int iters = base < t1 ? static_cast<int>((t1 - base + kStride - 1) / kStride) : 0;
    if (!(kEarly && t0 == first)) issue(A, base, t0, t1);
    for (int it = 0; it < iters; it += 2) {
      issue(B, base + (it + 1) * kStride, t0, t1);
      consume(A);
      if (it + 1 >= iters) break;
      issue(A, base + (it + 2) * kStride, t0, t1);
      consume(B);
    }
  }

  if (gl == 0) {
    s_m[slot] = run.m;
    s_l[slot] = run.l;
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i)
#pragma unroll
    for (int e = 0; e < VW; ++e) s_acc[slot * G * kPerLane + (gl + G * i) * VW + e] = run.acc[i][e];
  __syncthreads();

  float* rec = a.part + (static_cast<int64_t>(h) * a.splits + split) * (a.hd + 2);
  float big = -INFINITY;
  for (int t = 0; t < kSlots; ++t) big = fmaxf(big, s_m[t]);
  for (int e = threadIdx.x; e < a.hd; e += kBlock) {
    float total = 0.0f, sum = 0.0f;
    if (big != -INFINITY) {
      for (int t = 0; t < kSlots; ++t) {
        if (s_m[t] == -INFINITY) continue;
        const float wgt = exp_shift(s_m[t], big);
        total += s_l[t] * wgt;
        sum += s_acc[t * G * kPerLane + e] * wgt;
      }
    }
    rec[2 + e] = sum;
    if (e == 0) {
      rec[0] = big;
      rec[1] = total;
    }
  }
}

// One workgroup per (head, 64-element slice of the head). Wave 0 reads the
// splits' (m, l) pairs (SPLITS / 64 per lane) and turns them into weights
// 2^((m_s - M) log2 e) in LDS; then wave w sums splits w, w + 4, ... of the
// slice's weighted value records, with all SPLITS / 4 loads per lane issued
// together (indices clamped, weight 0 past `splits`); the four wave
// partials add in wave order. SPLITS is 64 or 128, the smallest that holds
// `splits`, so a short cache does not pay for 128 record loads.
template <int SPLITS>
__global__ __launch_bounds__(kBlock) void attend_merge(const float* __restrict__ part, int hd, int splits,
                                                       float* __restrict__ out) {
  constexpr int kPerWave = SPLITS / kWavesPerBlock;
  constexpr int kPerLane = SPLITS / kWave;
  __shared__ float s_w[SPLITS];
  __shared__ float s_total;
  __shared__ float s_red[kWavesPerBlock][kWave];
  const int slices = (hd + kWave - 1) / kWave;
  const int h = blockIdx.x / slices;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int e = (blockIdx.x - h * slices) * kWave + lane;
  const int ec = e < hd ? e : hd - 1;
  const int64_t rec_len = hd + 2;
  const float* recs = part + static_cast<int64_t>(h) * splits * rec_len;
  // Every load is issued before the first is used: wave 0's (m, l) pairs
  // first (a wave's loads complete in order, and the weights are formed from
  // them while the value records are still arriving), then the value
  // records.
  float m[kPerLane], l[kPerLane];
  if (wave == 0) {
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
      const int sp = lane + kWave * k;
      const int sc = sp < splits ? sp : splits - 1;
      m[k] = recs[sc * rec_len];
      l[k] = recs[sc * rec_len + 1];
    }
  }
  float vals[kPerWave];
#pragma unroll
  for (int r = 0; r < kPerWave; ++r) {
    const int sp = wave + kWavesPerBlock * r;
    vals[r] = recs[(sp < splits ? sp : splits - 1) * rec_len + 2 + ec];
  }
  if (wave == 0) {
    float big = -INFINITY;
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
      const int sp = lane + kWave * k;
      m[k] = sp < splits ? m[k] : -INFINITY;
      big = fmaxf(big, m[k]);
    }
    big = wave_max(big);
    float tl = 0.0f;
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
      const float w = (m[k] == -INFINITY || big == -INFINITY) ? 0.0f : exp_shift(m[k], big);
      s_w[lane + kWave * k] = w;
      tl = k == 0 ? w * l[k] : fmaf(w, l[k], tl);
    }
    const float total = wave_sum(tl);
    if (lane == 0) s_total = total;
  }
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int r = 0; r < kPerWave; ++r) {
    const int sp = wave + kWavesPerBlock * r;
    if (sp < splits) acc = fmaf(s_w[sp], vals[r], acc);
  }
  s_red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && e < hd) {
    const float total = s_total;
    const float sum = (s_red[0][lane] + s_red[1][lane]) + (s_red[2][lane] + s_red[3][lane]);
    out[static_cast<int64_t>(h) * hd + e] = total > 0.0f ? sum / total : 0.0f;
  }
}

// Splits per head: about 2048 workgroups (8 per CU) at every head count, but
// no split under 64 KB of key and value rows at a full cache, and at most
// 128. Measured at 10 heads of 128 against the 64 splits of a 1024-workgroup
// target: 6-7% faster for an fp32 cache at 8192 and 32768 positions (128
// splits), and for a bf16 cache the same at 8192 (64 splits), 4% faster at
// 32768 and 9% faster at 2048 (16 splits); an fp32 cache at 2048 positions
// (32 splits) was 4% slower. Halving the 64 KB floor (128 splits for a bf16
// cache at 8192 positions) was 11% slower (12.95 to 14.4 us).
int attend_splits(int64_t heads, int64_t hd, int64_t capacity, int64_t elem_bytes) {
  int64_t s = (2048 + heads - 1) / heads;
  int64_t min_keys = 65536 / (2 * hd * elem_bytes);
  if (min_keys < 32) min_keys = 32;
  const int64_t by_keys = (capacity + min_keys - 1) / min_keys;
  if (s > by_keys) s = by_keys;
  if (s > kMaxSplits) s = kMaxSplits;
  return static_cast<int>(s < 1 ? 1 : s);
}


template <class TC, int VW, int G, int VPL, int U, bool kRope>
void launch_partial(hipStream_t s, const AttendArgs& a, int64_t heads) {
  const unsigned blocks = static_cast<unsigned>(heads * a.splits);
  if constexpr (kRope) {
    if (a.segs != nullptr) {
      attend_partial<TC, VW, G, VPL, U, true, false, true><<<blocks, kBlock, 0, s>>>(a);
      return;
    }
  }
  if (kRope && a.mask == nullptr) {
    attend_partial<TC, VW, G, VPL, U, kRope, kRope><<<blocks, kBlock, 0, s>>>(a);
  } else {
    attend_partial<TC, VW, G, VPL, U, kRope, false><<<blocks, kBlock, 0, s>>>(a);
  }
}

// Lanes per key and keys per batch, with 16-byte chunks (4 fp32 or 8 bf16
// cache elements per lane). Up to 8192 positions two keys per batch (the
// split's keys are few, so fewer dead loads and registers win); beyond, four
// keys per batch and, where a key spans 32 chunks, 16 lanes of two chunks
// each. Both depend on the capacity only, so a captured step keeps its launch
// shape at every position.
template <class TC, bool kRope>
void launch_attend_vec(hipStream_t s, const AttendArgs& a, int64_t heads) {
  constexpr int VW = kVec<TC>;
  const int nvec = a.hd / VW;
  const bool long_ctx = a.capacity > 8192;
  if (nvec <= 1) launch_partial<TC, VW, 1, 1, 2, kRope>(s, a, heads);
  else if (nvec <= 2) launch_partial<TC, VW, 2, 1, 2, kRope>(s, a, heads);
  else if (nvec <= 4) launch_partial<TC, VW, 4, 1, 2, kRope>(s, a, heads);
  else if (nvec <= 8) launch_partial<TC, VW, 8, 1, 2, kRope>(s, a, heads);
  else if (nvec <= 16) {
    if (long_ctx) launch_partial<TC, VW, 16, 1, 4, kRope>(s, a, heads);
    else launch_partial<TC, VW, 16, 1, 2, kRope>(s, a, heads);
  } else if (nvec <= 32) {
    if (long_ctx) launch_partial<TC, VW, 16, 2, 4, kRope>(s, a, heads);
    else launch_partial<TC, VW, 32, 1, 2, kRope>(s, a, heads);
  } else {
    if (long_ctx) launch_partial<TC, VW, 64, 1, 4, kRope>(s, a, heads);
    else launch_partial<TC, VW, 64, 1, 2, kRope>(s, a, heads);
  }
}

template <class TC, bool kRope>
void launch_attend_any(hipStream_t s, const AttendArgs& a, int64_t heads) {
  if (a.hd <= 64) launch_partial<TC, 1, 64, 1, 2, kRope>(s, a, heads);
  else if (a.hd <= 128) launch_partial<TC, 1, 64, 2, 2, kRope>(s, a, heads);
  else launch_partial<TC, 1, 64, 4, 2, kRope>(s, a, heads);
}

void launch_merge(hipStream_t s, const AttendArgs& a, int64_t heads, float* out) {
  const unsigned blocks = static_cast<unsigned>(heads * ((a.hd + kWave - 1) / kWave));
  if (a.splits <= kWave) {
    attend_merge<kWave><<<blocks, kBlock, 0, s>>>(a.part, a.hd, a.splits, out);
  } else {
    attend_merge<kMaxSplits><<<blocks, kBlock, 0, s>>>(a.part, a.hd, a.splits, out);
  }
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

namespace uocr_rocm {
namespace {

template <class TC>
int append_entry(const char* what, void* stream, TC* cache, const float* row, int64_t width,
                 const uocr_rocm_step_state* state, int64_t capacity) {
  UOCR_REQUIRE(width >= 0, what, "width must be >= 0");
  if (width == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(cache != nullptr && row != nullptr && state != nullptr, what, "null pointer");
  UOCR_REQUIRE(width < (int64_t{1} << 36), what, "width too large");
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  if (width % 4 == 0 && aligned16(row) && (reinterpret_cast<uintptr_t>(cache) & (4 * sizeof(TC) - 1)) == 0) {
    const unsigned blocks = static_cast<unsigned>((width / 4 + kBlock - 1) / kBlock);
    append_k<TC, 4><<<blocks, kBlock, 0, s>>>(cache, row, width, state, capacity);
  } else {
    const unsigned blocks = static_cast<unsigned>((width + kBlock - 1) / kBlock);
    append_k<TC, 1><<<blocks, kBlock, 0, s>>>(cache, row, width, state, capacity);
  }
  return check_launch(what);
}

int check_attend(const char* what, int64_t heads, int64_t hd, int64_t capacity) {
  UOCR_REQUIRE(hd <= kMaxHeadDim, what, "head dim above 256");
  UOCR_REQUIRE(heads < (int64_t{1} << 24), what, "too many heads");
  UOCR_REQUIRE(capacity >= 1, what, "capacity must be >= 1");
  return UOCR_ROCM_OK;
}

template <class TC, bool kRope>
int attend_entry(const char* what, void* stream, AttendArgs a, int64_t heads, float* out) {
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  if (a.hd % kVec<TC> == 0 && aligned16(a.q) && aligned16(a.k) && aligned16(a.v)) {
    launch_attend_vec<TC, kRope>(s, a, heads);
  } else {
    launch_attend_any<TC, kRope>(s, a, heads);
  }
  if (const int st = check_launch(what); st != UOCR_ROCM_OK) return st;
  if (out == nullptr) return UOCR_ROCM_OK;  // the records stay for a merging consumer
  launch_merge(s, a, heads, out);
  return check_launch(what);
}

template <class TC>
int attend_plain(const char* what, void* stream, const float* q, const TC* k_cache, const TC* v_cache, int64_t heads,
                 int64_t hd, const float* mask, float scale, const uocr_rocm_step_state* state, float* scratch,
                 int64_t capacity, float* out) {
  UOCR_REQUIRE(heads >= 0 && hd >= 0, what, "heads and hd must be >= 0");
  if (heads == 0 || hd == 0) return UOCR_ROCM_OK;
  if (const int st = check_attend(what, heads, hd, capacity)) return st;
  UOCR_REQUIRE(q != nullptr && k_cache != nullptr && v_cache != nullptr && state != nullptr && scratch != nullptr &&
                   out != nullptr,
               what, "null pointer");
  AttendArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.mask = mask;
  a.part = scratch;
  a.state = state;
  a.width = heads * hd;
  a.capacity = capacity;
  a.scale = scale;
  a.hd = static_cast<int>(hd);
  a.splits = attend_splits(heads, hd, capacity, sizeof(TC));
  return attend_entry<TC, false>(what, stream, a, heads, out);
}

template <class TC>
int attend_rope(const char* what, void* stream, const float* q, const float* k_row, const float* v_row, TC* k_cache,
                TC* v_cache, int64_t heads, int64_t hd, const float* mask, float scale,
                const uocr_rocm_step_state* state, const float* inv_tok, int64_t n_tok, const float* inv_page,
                int64_t page_mod, float* scratch, int64_t capacity, float* out) {
  UOCR_REQUIRE(heads >= 0 && hd >= 0, what, "heads and hd must be >= 0");
  if (heads == 0 || hd == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(hd % 2 == 0, what, "head dim must be even and at most 256");
  if (const int st = check_attend(what, heads, hd, capacity)) return st;
  UOCR_REQUIRE(n_tok >= 0 && n_tok <= hd / 2, what, "n_tok must be in [0, hd / 2]");
  UOCR_REQUIRE(n_tok == 0 || inv_tok != nullptr, what, "null inv_tok");
  UOCR_REQUIRE(n_tok == hd / 2 || inv_page != nullptr, what, "null inv_page");
  UOCR_REQUIRE(q != nullptr && k_row != nullptr && v_row != nullptr && k_cache != nullptr && v_cache != nullptr &&
                   state != nullptr && scratch != nullptr && out != nullptr,
               what, "null pointer");
  AttendArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.mask = mask;
  a.part = scratch;
  a.state = state;
  a.width = heads * hd;
  a.capacity = capacity;
  a.scale = scale;
  a.hd = static_cast<int>(hd);
  a.splits = attend_splits(heads, hd, capacity, sizeof(TC));
  a.k_row = k_row;
  a.v_row = v_row;
  a.k_out = k_cache;
  a.v_out = v_cache;
  a.inv_tok = inv_tok;
  a.inv_page = inv_page;
  a.page_mod = page_mod;
  a.n_tok = static_cast<int>(n_tok);
  return attend_entry<TC, true>(what, stream, a, heads, out);
}

template <class TC>
int attend_rope_segments(const char* what, void* stream, const float* q, const float* k_row, const float* v_row,
                         TC* k_cache, TC* v_cache, int64_t heads, int64_t hd, const int32_t* segments,
                         int64_t max_live, float scale, const uocr_rocm_step_state* state, const float* inv_tok,
                         int64_t n_tok, const float* inv_page, int64_t page_mod, float* scratch, int64_t capacity,
                         float* out) {
  UOCR_REQUIRE(heads >= 0 && hd >= 0, what, "heads and hd must be >= 0");
  if (heads == 0 || hd == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(hd % 2 == 0, what, "head dim must be even and at most 256");
  if (const int st = check_attend(what, heads, hd, capacity)) return st;
  UOCR_REQUIRE(max_live >= 1 && max_live <= capacity, what, "max_live must be in [1, capacity]");
  UOCR_REQUIRE(n_tok >= 0 && n_tok <= hd / 2, what, "n_tok must be in [0, hd / 2]");
  UOCR_REQUIRE(n_tok == 0 || inv_tok != nullptr, what, "null inv_tok");
  UOCR_REQUIRE(n_tok == hd / 2 || inv_page != nullptr, what, "null inv_page");
  UOCR_REQUIRE(q != nullptr && k_row != nullptr && v_row != nullptr && k_cache != nullptr && v_cache != nullptr &&
                   segments != nullptr && state != nullptr && scratch != nullptr,
               what, "null pointer");
  AttendArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.mask = nullptr;
  a.segs = segments;
  a.part = scratch;
  a.state = state;
  a.width = heads * hd;
  a.capacity = capacity;
  a.scale = scale;
  a.hd = static_cast<int>(hd);
  a.splits = segment_splits(max_live);
  a.k_row = k_row;
  a.v_row = v_row;
  a.k_out = k_cache;
  a.v_out = v_cache;
  a.inv_tok = inv_tok;
  a.inv_page = inv_page;
  a.page_mod = page_mod;
  a.n_tok = static_cast<int>(n_tok);
  return attend_entry<TC, true>(what, stream, a, heads, out);
}

}  // namespace

// uocr_rocm_attend_step's body under a caller-chosen name (the entry point
// that allocates nothing reports its errors under its own name).
int attend_step_f32(const char* what, void* stream, const float* q, const float* k_cache, const float* v_cache,
                    int64_t heads, int64_t hd, const float* mask, float scale, const uocr_rocm_step_state* state,
                    float* scratch, int64_t capacity, float* out) {
  return attend_plain(what, stream, q, k_cache, v_cache, heads, hd, mask, scale, state, scratch, capacity, out);
}

}  // namespace uocr_rocm

extern "C" {

int uocr_rocm_append_step(void* stream, float* cache, const float* row, int64_t width,
                          const uocr_rocm_step_state* state, int64_t capacity) {
  return append_entry("uocr_rocm_append_step", stream, cache, row, width, state, capacity);
}

int uocr_rocm_append_step_bf16(void* stream, uint16_t* cache, const float* row, int64_t width,
                               const uocr_rocm_step_state* state, int64_t capacity) {
  return append_entry("uocr_rocm_append_step_bf16", stream, cache, row, width, state, capacity);
}

int64_t uocr_rocm_attend_scratch_floats(int64_t heads, int64_t hd, int64_t capacity) {
  if (heads <= 0 || hd <= 0 || capacity <= 0) return 0;
  // An fp32 cache has the most splits; a bf16 cache uses at most as many.
  return heads * attend_splits(heads, hd, capacity, sizeof(float)) * (hd + 2);
}

int uocr_rocm_attend_step(void* stream, const float* q, const float* k_cache, const float* v_cache, int64_t heads,
                          int64_t hd, const float* mask, float scale, const uocr_rocm_step_state* state,
                          float* scratch, int64_t capacity, float* out) {
  return attend_plain("uocr_rocm_attend_step", stream, q, k_cache, v_cache, heads, hd, mask, scale, state, scratch,
                      capacity, out);
}

int uocr_rocm_attend_step_bf16(void* stream, const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                               int64_t heads, int64_t hd, const float* mask, float scale,
                               const uocr_rocm_step_state* state, float* scratch, int64_t capacity, float* out) {
  return attend_plain("uocr_rocm_attend_step_bf16", stream, q, k_cache, v_cache, heads, hd, mask, scale, state,
                      scratch, capacity, out);
}

int uocr_rocm_attend_rope_kv_step(void* stream, const float* q, const float* k_row, const float* v_row,
                                  float* k_cache, float* v_cache, int64_t heads, int64_t hd, const float* mask,
                                  float scale, const uocr_rocm_step_state* state, const float* inv_tok, int64_t n_tok,
                                  const float* inv_page, int64_t page_mod, float* scratch, int64_t capacity,
                                  float* out) {
  return attend_rope("uocr_rocm_attend_rope_kv_step", stream, q, k_row, v_row, k_cache, v_cache, heads, hd, mask,
                     scale, state, inv_tok, n_tok, inv_page, page_mod, scratch, capacity, out);
}

int64_t uocr_rocm_attend_segments_scratch_floats(int64_t heads, int64_t hd, int64_t max_live) {
  if (heads <= 0 || hd <= 0 || max_live <= 0) return 0;
  return heads * segment_splits(max_live) * (hd + 2);
}

int uocr_rocm_attend_rope_kv_step_segments(void* stream, const float* q, const float* k_row, const float* v_row,
                                           float* k_cache, float* v_cache, int64_t heads, int64_t hd,
                                           const int32_t* segments, int64_t max_live, float scale,
                                           const uocr_rocm_step_state* state, const float* inv_tok, int64_t n_tok,
                                           const float* inv_page, int64_t page_mod, float* scratch, int64_t capacity,
                                           float* out) {
  return attend_rope_segments("uocr_rocm_attend_rope_kv_step_segments", stream, q, k_row, v_row, k_cache, v_cache,
                              heads, hd, segments, max_live, scale, state, inv_tok, n_tok, inv_page, page_mod, scratch,
                              capacity, out);
}

int uocr_rocm_attend_rope_kv_step_segments_bf16(void* stream, const float* q, const float* k_row, const float* v_row,
                                                uint16_t* k_cache, uint16_t* v_cache, int64_t heads, int64_t hd,
                                                const int32_t* segments, int64_t max_live, float scale,
                                                const uocr_rocm_step_state* state, const float* inv_tok,
                                                int64_t n_tok, const float* inv_page, int64_t page_mod,
                                                float* scratch, int64_t capacity, float* out) {
  return attend_rope_segments("uocr_rocm_attend_rope_kv_step_segments_bf16", stream, q, k_row, v_row, k_cache,
                              v_cache, heads, hd, segments, max_live, scale, state, inv_tok, n_tok, inv_page, page_mod,
                              scratch, capacity, out);
}

int uocr_rocm_attend_rope_kv_step_bf16(void* stream, const float* q, const float* k_row, const float* v_row,
                                       uint16_t* k_cache, uint16_t* v_cache, int64_t heads, int64_t hd,
                                       const float* mask, float scale, const uocr_rocm_step_state* state,
                                       const float* inv_tok, int64_t n_tok, const float* inv_page, int64_t page_mod,
                                       float* scratch, int64_t capacity, float* out) {
  return attend_rope("uocr_rocm_attend_rope_kv_step_bf16", stream, q, k_row, v_row, k_cache, v_cache, heads, hd,
                     mask, scale, state, inv_tok, n_tok, inv_page, page_mod, scratch, capacity, out);
}

}  // extern "C"
