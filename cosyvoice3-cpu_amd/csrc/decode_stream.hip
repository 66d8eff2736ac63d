// The Qwen2 decode step as one launch over per-workgroup weight streams
// (cv3cpu/models/qwen2.py:139-179, cv3cpu/models/llm.py:68-77,112-123; the
// quantised GEMVs are quant.py:172-204 at m = 1).
//
// Why a second one-launch step.  Batch-1 decode is a chain of five grid-wide
// dependencies per layer (x -> [q;k;v] -> attention partials -> x_mid -> h -> x).
// When each phase also fetches its weights after its input arrives, the fetch
// sits on that chain.  Here the weights never do:
//
//  * A host plan splits every layer's matrices into units of 16 output rows and
//    assigns them to the workgroups (one per CU): [q;k;v] in rotary pairs (rows j
//    and j + dh/2 of a head in one unit), o_proj, [gate; up] pairs, down in four
//    K quarters (16 rows x I/4), and the LM head.  A pack kernel lays each
//    workgroup's units out as one contiguous stream per layer: its per-row scales,
//    then its tiles in the order the phases use them.
//  * A tile is 16 rows x 64 codes in the B-operand order of
//    v_mfma_i32_16x16x64_i8 (lane l: row l % 16, codes 16 (l / 16) .. +16 of the
//    64), 1 KB.  The ninth wave of each workgroup only streams: it DMAs tiles
//    global -> LDS (global_load_lds_dwordx4) into a 96-slot ring, as far ahead as
//    the ring allows, and publishes how far it got; the eight compute waves mark
//    units done so it can reuse their slots.  A phase finds its tiles in LDS.
//  * The dot products run on the matrix cores, exactly: the activation vector v
//    is split into four signed base-128 digit planes against a shared power of two
//    (X = rint(v 2^(27 - E)), |v| < 2^E, X = d0 + 128 d1 + 128^2 d2 + 128^3 d3 with
//    d_p in [-64, 64]).  An MFMA of the planes (A rows 0..3) with a tile gives each
//    row's four plane sums in int32, exact; they combine in float64 into
//    sum_k q_k X_k exactly, times 2^(E - 27) and the row's scale.  The result is
//    the dot product of the int8 row with v rounded to 27 bits below its largest
//    element (the reference: v in float32 with float32 accumulation), so rows
//    cost no per-code VALU work at all.  Block-64 scales (balanced profile) are
//    applied per tile, since a tile is one scale block.
//
// Exchanges between the phases are the epoch-tagged 64-bit words of the first
// one-launch step (value | epoch << 32, relaxed agent-scope atomics, double
// buffered by layer parity, bounded waits that set the error flag).  The down
// projection's four K quarters each publish a partial x; readers add them in a
// fixed order, (p0 + p1) + (p2 + p3), with the residual x_mid inside p0.
#include <algorithm>
#include <string>
#include <vector>

#include "common.hpp"
#include "decode_common.hpp"

using namespace cv3;

namespace {


constexpr int kST = 576;                 // threads: 8 compute waves + the loader wave
constexpr int kSC = 8;                   // compute waves
constexpr int kSRing = 96;               // LDS ring of 1 KB tiles
constexpr int kSSb = 3;                  // scale buffers (layer % 3)
constexpr int kSSbBytes = 3072;          // bytes per scale buffer
constexpr int kSQ = 4;                   // K quarters of the down projection
constexpr int kSPW = 24;                 // int64 per workgroup in the plan table
constexpr int kSRX = 2, kSRM = 2, kSRH = 1, kSRP = 1;  // replicas of the exchanged vectors
constexpr int kSInflight = 40;           // DMA instructions the loader keeps in flight
constexpr int kSBig = 7680;              // floats: attention partials (C) with x rows and chunk weights, h quarter (E), x quarters
constexpr int kSPlane = 1280;            // bytes per digit plane (K <= 1280)

// plan table fields (int64 each)
enum {
  P_A, P_C, P_ND, P_D0, P_D1, P_NE, P_E0, P_E1, P_NH, P_H0, P_H1,
  P_SB, P_SBH,       // scale bytes of a layer region / of the head region
  P_NL, P_NHT,       // tiles per layer / in the head region
  P_OFF,             // byte offset of this workgroup's stream
  P_STRIDE,          // bytes per layer region
  P_HOFF,            // byte offset of the head region
  P_SPAD, P_SPADH,   // scale bytes padded (tiles start there) per layer / head region
};

enum { U_A, U_C, U_D, U_E, U_H };

struct SGeo {
  int L, D, H, Hk, dh, I, V, G;
  int KB;   // D / 64: tiles per 16-row unit of a D-wide row
  int KBQ;  // I / (64 kSQ): tiles per down quarter
  int R;    // (H + 2 Hk) dh
  int nA, nC, nD, nE, nHd;
  int b64;  // block-64 float16 scales (1) or one scale per row (0)
  int Bbase;  // first attention-item workgroup
};

__host__ __device__ inline int unit_tiles(const SGeo& g, int type) {
  return type == U_D ? 2 * g.KB : type == U_E ? g.KBQ : g.KB;
}
// bytes of a unit's scales in a stream: per row, one float per row set; block-64, one half per (tile, row)
__host__ __device__ inline int unit_scale_bytes(const SGeo& g, int type) {
  const int sets = type == U_D ? 2 : 1;
  return g.b64 ? unit_tiles(g, type) * 16 * 2 : sets * 16 * 4;
}

// Source of column j of tile kt of a unit: matrix (0 qkv, 1 o, 2 gate_up, 3 down, 4 head), row, k-block.
struct TileSrc {
  int mat, row, kb;
};
__host__ __device__ inline TileSrc tile_src(const SGeo& g, int type, int u, int kt, int j) {
  TileSrc s{0, 0, kt};
  if (type == U_A) {
    const int upk = g.dh / 16, hd = u / upk, sub = u % upk;
    s.mat = 0;
    s.row = hd * g.dh + sub * 8 + (j & 7) + (j >= 8 ? g.dh / 2 : 0);
  } else if (type == U_C) {
    s.mat = 1;
    s.row = u * 16 + j;
  } else if (type == U_D) {
    s.mat = 2;
    s.row = (kt < g.KB ? 0 : g.I) + u * 16 + j;
    s.kb = kt % g.KB;
  } else if (type == U_E) {
    s.mat = 3;
    s.row = (u / kSQ) * 16 + j;
    s.kb = (u % kSQ) * g.KBQ + kt;
  } else {
    s.mat = 4;
    s.row = min(u * 16 + j, g.V - 1);
  }
  return s;
}

// The units of one region of a workgroup's stream, in stream order.
struct Units {
  int n;
  int type[6], id[6];
};
__host__ __device__ inline Units region_units(const int64_t* P, bool head) {
  Units r{};
  auto add = [&](int t, int64_t u) {
    r.type[r.n] = t;
    r.id[r.n] = (int)u;
    ++r.n;
  };
  if (head) {
    for (int i = 0; i < P[P_NH]; ++i) add(U_H, P[P_H0 + i]);
  } else {
    if (P[P_A] >= 0) add(U_A, P[P_A]);
    if (P[P_C] >= 0) add(U_C, P[P_C]);
    for (int i = 0; i < P[P_ND]; ++i) add(U_D, P[P_D0 + i]);
    for (int i = 0; i < P[P_NE]; ++i) add(U_E, P[P_E0 + i]);
  }
  return r;
}

// ---------------------------------------------------------------------------
// Pack: one workgroup per (stream workgroup, region); region L is the head.
// ---------------------------------------------------------------------------
struct PackArgs {
  SGeo g;
  const int8_t* w[5];      // qkv, o, gate_up, down, head codes
  const void* s[5];        // their scales
  int64_t rows[5], kp[5], nb[5];
  int sf16[5];
  const int64_t* plan;
  uint8_t* out;
};

__global__ __launch_bounds__(256) void k_stream_pack(PackArgs a) {
  const SGeo& g = a.g;
  const int w = blockIdx.x, l = blockIdx.y;
  const bool head = l == g.L;
  const int64_t* P = a.plan + (int64_t)w * kSPW;
  const Units u = region_units(P, head);
  uint8_t* dst = a.out + P[P_OFF] + (head ? P[P_HOFF] : (int64_t)l * P[P_STRIDE]);
  const int lay = head ? 0 : l;
  // scales
  int soff = 0;
  for (int i = 0; i < u.n; ++i) {
    const int nt = unit_tiles(g, u.type[i]);
    if (g.b64) {
      for (int e = threadIdx.x; e < nt * 16; e += blockDim.x) {
        const int kt = e / 16, j = e % 16;
        const TileSrc s = tile_src(g, u.type[i], u.id[i], kt, j);
        const int64_t si = ((int64_t)lay * a.rows[s.mat] + s.row) * a.nb[s.mat] + s.kb;
        reinterpret_cast<__half*>(dst + soff)[e] = reinterpret_cast<const __half*>(a.s[s.mat])[si];
      }
    } else {
      const int sets = u.type[i] == U_D ? 2 : 1;
      for (int e = threadIdx.x; e < sets * 16; e += blockDim.x) {
        const TileSrc s = tile_src(g, u.type[i], u.id[i], (e / 16) * g.KB, e % 16);
        const int64_t si = ((int64_t)lay * a.rows[s.mat] + s.row) * a.nb[s.mat];
        reinterpret_cast<float*>(dst + soff)[e] =
            a.sf16[s.mat] ? __half2float(reinterpret_cast<const __half*>(a.s[s.mat])[si])
                          : reinterpret_cast<const float*>(a.s[s.mat])[si];
      }
    }
    soff += unit_scale_bytes(g, u.type[i]);
  }
  // tiles: 64 lanes x 16 bytes each
  uint8_t* tiles = dst + (head ? P[P_SPADH] : P[P_SPAD]);
  const int ntiles = (int)(head ? P[P_NHT] : P[P_NL]);
  for (int it = threadIdx.x; it < ntiles * 64; it += blockDim.x) {
    const int t = it / 64, lane = it % 64;
    int ui = 0, t0 = 0;
    while (t - t0 >= unit_tiles(g, u.type[ui])) t0 += unit_tiles(g, u.type[ui++]);
    const TileSrc s = tile_src(g, u.type[ui], u.id[ui], t - t0, lane % 16);
    const int8_t* src = a.w[s.mat] + ((int64_t)lay * a.rows[s.mat] + s.row) * a.kp[s.mat] + s.kb * 64 + (lane / 16) * 16;
    *reinterpret_cast<u32x4*>(tiles + (int64_t)t * 1024 + lane * 16) = *reinterpret_cast<const u32x4*>(src);
  }
}

// ---------------------------------------------------------------------------
// The step.
// ---------------------------------------------------------------------------
struct SArgs {
  const uint8_t* packed;
  const int64_t* plan;
  SGeo g;
  const float *ln1, *ln2, *norm, *qkv_bias, *head_bias, *rope_cos, *rope_sin;
  QW emb;
  float eps, scale;
  float *k_cache, *v_cache;
  int64_t cap;
  int64_t *pos, *token, *history;
  float *x, *logits;
  uint64_t *xb, *qkvb, *pb, *mb, *hb, *arg;
  int64_t sx, sp, sm, sh;  // words between replicas
  int64_t* err;
  uint32_t epoch_base;
  int select;
};

struct SShared {
  uint32_t loaded;  // loader: DMA instructions known to have landed
  uint32_t udone;   // compute: units whose tiles are no longer read
  uint32_t bar;     // compute-wave barrier counter
  uint32_t fail;    // a wait gave up
};

// Workgroup memory of the step, at file scope: every access names its array, so the
// compiler can tell the loader's DMA targets (s_ring, s_sbuf) from the other LDS traffic.
__shared__ __align__(16) uint8_t s_ring[kSRing * 1024];    // tiles, as the loader streams them
__shared__ __align__(16) uint8_t s_sbuf[kSSb * kSSbBytes];  // scales of layers l % 3
__shared__ __align__(16) float s_xin[1024];                 // x of the layer
__shared__ __align__(16) float s_xmid[1024];                // C: attention output; D, E: x_mid
__shared__ __align__(16) int8_t s_pln[4 * kSPlane];         // digit planes of the current vector
__shared__ __align__(16) int8_t s_zero[16];                 // the MFMA A rows above the planes
__shared__ __align__(16) float s_big[kSBig];                // partials, h quarter, x quarters
__shared__ float s_red[2 * kSC + 8];
__shared__ float s_hbv[kSC];
__shared__ int s_hbi[kSC];
__shared__ uint64_t s_hbk[kSC];
__shared__ SShared s_sh;
__shared__ uint32_t s_wait[kSC * 8];  // per compute wave and phase: the sleep before polling (ticks)

__device__ __forceinline__ uint32_t lds_load(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Marks this workgroup's step as failed: every compute wave leaves at its next barrier or
// wait, the loader at its next idle check, and the host sees the error flag.
__device__ __forceinline__ void give_up(int64_t* err) {
  __hip_atomic_store(&s_sh.fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  atomicOr(reinterpret_cast<unsigned long long*>(err), 1ull);
}

// Barrier of the eight compute waves (the loader wave never joins one): LDS writes
// before it are visible to every compute wave after it.  False once the step has
// failed (a wave that left early never arrives); bounded like every other wait.
__device__ __forceinline__ bool cbar(uint32_t tgt, int64_t* err) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(&s_sh.bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  for (int spins = 0; lds_load(&s_sh.bar) < tgt; ++spins) {
    if (lds_load(&s_sh.fail)) return false;
    if (spins >= kPSpin) {
      give_up(err);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");
  return !lds_load(&s_sh.fail);
}
#define CBAR()                     \
  do {                             \
    tgt += kSC;                    \
    if (!cbar(tgt, a.err)) return; \
  } while (0)

// Two ranges of exchange words, each with its own epoch, read as one vector: words [0, n0) from p0, then
// n1 words from p1 in rows of 2^sh1 words, st1 words apart (sh1 = 30: one contiguous range).
struct Segs {
  const uint64_t* p0;
  const uint64_t* p1;
  int n0, n1;
  uint32_t e0, e1;
  int sh1, st1;
};

constexpr int kGW = 8;  // words per thread per pass of a collective read (4096 per pass)

// Polls one exchange word until it carries epoch e (bounded; false on failure or when another wave gave up).
__device__ __forceinline__ bool poll_word(const uint64_t* p, uint32_t e, uint64_t& wv, int& spins,
                                          const int64_t* err) {
  for (spins = 0; spins < kPSpin; ++spins) {
    wv = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((uint32_t)(wv >> 32) == e) return true;
    if ((spins & 255) == 255 &&
        (lds_load(&s_sh.fail) || __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0))
      return false;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// Waits until DMA instruction `instr` of this workgroup's stream has landed in LDS.
__device__ __forceinline__ bool wait_loaded(uint32_t instr, int64_t* err) {
  for (int spins = 0; lds_load(&s_sh.loaded) <= instr; ++spins) {
    if (lds_load(&s_sh.fail)) return false;
    if (spins >= kPSpin) {
      give_up(err);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

// A wave about to wait for a phase's input first sleeps for `target` wall-clock ticks (hundreds of workgroups
// polling from the start slow every exchange down; the layers take the same time, so the last layer's wait
// predicts this one).  The target adapts per wave and phase without feeding back on itself: when every word was
// already there at the first poll the wave slept too long and the target halves; otherwise it becomes three
// quarters of the whole wait (sleep included: the input came after the sleep ended).
constexpr uint32_t kSleepCap = 2000;  // ticks (100 MHz): 20 us
__device__ __forceinline__ void presleep(uint64_t t0, uint32_t target) {
  while (wall_clock64() - t0 < target) __builtin_amdgcn_s_sleep(10);
}
__device__ __forceinline__ uint32_t next_sleep(uint64_t t0, uint32_t target, bool overslept) {
  return overslept ? target / 2 : (uint32_t)min((wall_clock64() - t0) * 3 / 4, (uint64_t)kSleepCap);
}

enum { PH_A, PH_B, PH_C, PH_D, PH_E, PH_HEAD };

template <bool B64>
__global__ __launch_bounds__(kST) void k_dec_stream(SArgs a) {
  const SGeo& g = a.g;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int w = blockIdx.x;
  const int64_t* P = a.plan + (int64_t)w * kSPW;
  if (tid == 0) {
    s_sh.loaded = 0;
    s_sh.udone = 0;
    s_sh.bar = 0;
    s_sh.fail = 0;
  }
  if (tid < 4) reinterpret_cast<uint32_t*>(s_zero)[tid] = 0u;
  if (tid < kSC * 8) s_wait[tid] = 0u;
  __syncthreads();  // the only full-workgroup barrier: from here the loader runs on its own
  if (wave == kSC) {
    // ---- the loader wave.  Its DMAs target s_ring / s_sbuf and its own LDS accesses of s_sh
    // are plain loads and stores of that variable (a compiler barrier forces each poll to
    // read again): the compiler can then tell them apart and needs no wait for the DMAs in
    // flight before them (atomic, volatile or pointer-argument accesses make it wait for
    // every DMA, one latency per tile).  Every plan value it needs is read once, before
    // the loop: inside it the only global memory operations are the DMAs, so a wait on
    // vmcnt never waits for anything else. ----
    const int L = g.L;
    // units per layer in stream order: one A or C unit (or none), nd [gate; up] units, ne down units; a phase's
    // tiles are freed once all of its units are done
    const uint32_t nac = (P[P_A] >= 0 ? 1u : 0u) + (P[P_C] >= 0 ? 1u : 0u);
    const uint32_t nd = (uint32_t)P[P_ND], ne = (uint32_t)P[P_NE];
    const uint32_t upl = nac + nd + ne;
    const uint32_t tac = nac * (uint32_t)g.KB, td = nd * 2u * (uint32_t)g.KB;
    const uint32_t nl = (uint32_t)P[P_NL], nht = (uint32_t)P[P_NHT];
    const uint32_t sbl = (uint32_t)P[P_SB], sbh = (uint32_t)P[P_SBH];
    const uint32_t sl = (sbl + 1023u) / 1024u, shd = (sbh + 1023u) / 1024u;
    const uint8_t* const base = a.packed + P[P_OFF];
    const int64_t stride = P[P_STRIDE], hoff = P[P_HOFF], spad = P[P_SPAD], spadh = P[P_SPADH];
    __builtin_amdgcn_s_waitcnt(CV3_VMCNT(0));
    uint32_t issued = 0, landed = 0, idle = 0;
    for (uint32_t l = 0; l <= (uint32_t)L; ++l) {
      const bool head = l == (uint32_t)L;
      const uint32_t rs = head ? shd : sl, rn = head ? nht : nl, sbytes = head ? sbh : sbl;
      const uint8_t* const region = base + (head ? hoff : (int64_t)l * stride);
      const uint8_t* const tiles = region + (head ? spadh : spad);
      const uint32_t sdst = (l % kSSb) * kSSbBytes;
      const int64_t scale_ready = ((int64_t)l - 2) * upl;  // buffer l % 3 last held layer l - 3
      uint32_t slot = (l * nl) % kSRing;
      for (uint32_t r = 0; r < rs + rn;) {
        asm volatile("" ::: "memory");  // a fresh read every pass
        const uint32_t ud = s_sh.udone;
        bool ok;
        if (r < rs) {
          ok = (int64_t)ud >= scale_ready;
        } else {
          const uint32_t ul = ud / upl, ur = ud - ul * upl;
          const uint32_t freed = ul >= (uint32_t)L ? (uint32_t)L * nl
                                                   : ul * nl + (ur < nac ? 0u : ur < nac + nd ? tac : tac + td);
          ok = l * nl + (r - rs) < freed + kSRing;
        }
        if (!ok) {
          __builtin_amdgcn_s_waitcnt(CV3_VMCNT(0));
          landed = issued;
          s_sh.loaded = landed;
          asm volatile("" ::: "memory");
          if ((++idle & 255) == 0 &&
              (s_sh.fail || __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0))
            return;  // every DMA has landed (waited above)
          __builtin_amdgcn_s_sleep(1);
          continue;
        }
        if (r < rs) {
          if (r * 1024u + (uint32_t)lane * 16u < sbytes)
            __builtin_amdgcn_global_load_lds(region + r * 1024u + lane * 16, s_sbuf + sdst + r * 1024u, 16, 0, 0);
        } else {
          __builtin_amdgcn_global_load_lds(tiles + (int64_t)(r - rs) * 1024 + lane * 16, s_ring + slot * 1024, 16,
                                           0, 0);
          slot = slot + 1 == kSRing ? 0 : slot + 1;
        }
        ++r;
        ++issued;
        if (issued - landed > (uint32_t)kSInflight) {
          __builtin_amdgcn_s_waitcnt(CV3_VMCNT(kSInflight));
          landed = issued - kSInflight;
          s_sh.loaded = landed;
          asm volatile("" ::: "memory");
        }
      }
    }
    // no DMA may still be writing this workgroup's LDS when it ends
    __builtin_amdgcn_s_waitcnt(CV3_VMCNT(0));
    s_sh.loaded = issued;
    return;
  }

  // ---- the compute waves: one pass of the loop per (layer, phase); the collective read, the digit
  // planes and the MFMA unit appear once, so the kernel stays small ----
  uint32_t tgt = 0;  // compute-barrier target
  const int D = g.D, H = g.H, Hk = g.Hk, dh = g.dh, I = g.I, R = g.R, KB = g.KB, L = g.L;
  const uint32_t ebase = a.epoch_base;
  const int64_t pos = *a.pos;
  const int nact = (int)((pos + kPKeys) / kPKeys);
  const int ua = (int)P[P_A], uc = (int)P[P_C], nd = (int)P[P_ND], ne = (int)P[P_NE], nhu = (int)P[P_NH];
  const int nl = (int)P[P_NL];
  const int sl = (int)((P[P_SB] + 1023) / 1024), shd = (int)((P[P_SBH] + 1023) / 1024);
  const uint32_t per = (uint32_t)(sl + nl);
  const int tC0 = ua >= 0 ? KB : 0, tD0 = tC0 + (uc >= 0 ? KB : 0), tE0 = tD0 + 2 * KB * nd;
  const int sC = ua >= 0 ? unit_scale_bytes(g, U_A) : 0;
  const int sD = sC + (uc >= 0 ? unit_scale_bytes(g, U_C) : 0);
  const int sE = sD + nd * unit_scale_bytes(g, U_D);
  const bool isB = w >= g.Bbase && w < g.Bbase + H * kPChunks && ((w - g.Bbase) % kPChunks) < nact;
  const int qE = ne > 0 ? (int)P[P_E0] % kSQ : 0;  // the K quarter of this workgroup's down units
  const int KQ = I / kSQ;
  const int rx = w % kSRX, rm = w % kSRM, rh = w % kSRH;
  const int np = nact * H * kPPart;
  // row ids of this workgroup's [gate; up], down and head units (at most two of each, one per wave)
  const int ud0 = (int)P[P_D0], ud1 = (int)P[P_D1], ue0 = (int)P[P_E0], ue1 = (int)P[P_E1];
  const int uh0 = (int)P[P_H0], uh1 = (int)P[P_H1];

  for (int l = 0; l <= L; ++l) {
    const int par = l & 1;
    const uint32_t E = ebase + (uint32_t)l * 8u;
    const int sb = (l % kSSb) * kSSbBytes;
    const uint32_t lbase = (uint32_t)l * per + (uint32_t)sl;  // DMA instruction of this layer's tile 0
    const uint32_t pbase = (uint32_t)l * (uint32_t)nl;        // ring position of this layer's tile 0
    // x of the layer: four quarter partials of the previous layer's down projection
    const uint64_t* xq = a.xb + ((int64_t)(par ^ 1) * kSRX + rx) * a.sx;
    for (int ph = l == L ? PH_HEAD : PH_A; ph <= (l == L ? PH_HEAD : PH_E); ++ph) {
      // ---- this workgroup's part of the phase ----
      int nunits = 0;
      if (ph == PH_A) nunits = ua >= 0 ? 1 : 0;
      else if (ph == PH_B) nunits = isB ? 1 : 0;
      else if (ph == PH_C) nunits = uc >= 0 ? 1 : 0;
      else if (ph == PH_D) nunits = nd;
      else if (ph == PH_E) nunits = ne;
      else nunits = nhu;
      if (nunits == 0) continue;
      // ---- the phase's input: exchange words (and, for the attention item, the cached K / V rows) ----
      const int bh = isB ? (w - g.Bbase) / kPChunks : 0, bc = isB ? (w - g.Bbase) % kPChunks : 0;
      const int bg = bh / (H / Hk);
      const int kw = bc * kPKeys + 16 * wave, key = kw + (lane >> 2), qd = (lane & 3) * 16;
      const float* nw = ph == PH_A ? a.ln1 + (int64_t)l * D : ph == PH_D ? a.ln2 + (int64_t)l * D
                                                                          : ph == PH_HEAD ? a.norm : nullptr;
      const float4 wq = nw && tid < D / 4 ? reinterpret_cast<const float4*>(nw)[tid] : make_float4(1.f, 1.f, 1.f, 1.f);
      // operands of the phase's epilogue, fetched before the wait: the A unit's bias and rotary factors, the
      // head's bias
      const int jr = lane & 15;
      float ep0 = 0.f, ep1 = 1.f, ep2 = 0.f;
      if (ph == PH_A) {
        const int row = tile_src(g, U_A, ua, 0, jr).row, d = row % dh;
        ep0 = a.qkv_bias[(int64_t)l * R + row];
        if (row / dh < H + Hk) {
          ep1 = a.rope_cos[pos * dh + d];
          ep2 = a.rope_sin[pos * dh + d];
        }
      } else if (ph == PH_HEAD && a.head_bias && wave < nhu) {
        ep0 = a.head_bias[min((wave == 0 ? uh0 : uh1) * 16 + jr, g.V - 1)];  // rows past V are not stored
      }
      const uint64_t t_in = wall_clock64();
      const uint32_t prev = s_wait[wave * 8 + ph];
      if (ph == PH_B) {
        // ---- the attention item: K / V rows issued before the wait (they arrive while it polls), then q, k, v
        // of the head (one word per thread), then its own arithmetic, no tiles ----
        float4 kr[4];
        float vr[16];
        const int last = pos > 0 ? (int)pos - 1 : 0;  // cache rows before pos come from earlier launches
        const float* kbp = a.k_cache + ((int64_t)l * Hk + bg) * a.cap * dh;
        const float* vbp = a.v_cache + ((int64_t)l * Hk + bg) * a.cap * dh;
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[i] = reinterpret_cast<const float4*>(kbp + (int64_t)min(key, last) * dh + qd)[i];
#pragma unroll
        for (int t = 0; t < 16; ++t) vr[t] = vbp[(int64_t)min(kw + t, last) * dh + lane];
        presleep(t_in, prev);
        {
          const uint64_t* qb = a.qkvb + (int64_t)par * R;
          const int which = tid / dh, d = tid % dh;  // 0: q of head bh, 1: k, 2: v of group bg
          const uint64_t* src = qb + (which == 0 ? bh : which == 1 ? H + bg : H + Hk + bg) * dh + d;
          uint64_t wv = 0;
          int spun = 0;
          const bool ok = which >= 3 || poll_word(src, E, wv, spun, a.err);
          if (which < 3) s_big[tid] = __uint_as_float((uint32_t)wv);
          if (!ok) give_up(a.err);
          const uint32_t nxt = next_sleep(t_in, prev, __all(spun == 0));
          if (lane == 0) s_wait[wave * 8 + ph] = nxt;
          CBAR();
        }
        const float* qkv = s_big;
        const int ipos = (int)pos;
        if (key == ipos) {
#pragma unroll
          for (int i = 0; i < 4; ++i) kr[i] = reinterpret_cast<const float4*>(qkv + dh + qd)[i];
        }
        // scores in base-2 units: (q * scale) first (ops.py:292), then * log2(e)
        float sc = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 q4 = reinterpret_cast<const float4*>(qkv + qd)[i];
          sc = fmaf((q4.x * a.scale) * kLog2E, kr[i].x, sc);
          sc = fmaf((q4.y * a.scale) * kLog2E, kr[i].y, sc);
          sc = fmaf((q4.z * a.scale) * kLog2E, kr[i].z, sc);
          sc = fmaf((q4.w * a.scale) * kLog2E, kr[i].w, sc);
        }
        sc += __uint_as_float(dpp32<kDppXor1>(__float_as_uint(sc)));
        sc += __uint_as_float(dpp32<kDppXor2>(__float_as_uint(sc)));
        sc = key <= ipos ? sc : -INFINITY;
        const float mw = wave_max_dpp(sc);
        const float p = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sc - mw);
        const float lw = wave_sum_swap((lane & 3) == 0 ? p : 0.f);
        const float vnew = qkv[2 * dh + lane];
        const int tn = ipos - kw;
        float o = 0.f;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          const float pt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), 4 * t));
          o = fmaf(pt, t == tn ? vnew : vr[t], o);
        }
        float* ow = s_big + 4 * dh;  // [8 waves][dh], then m, l per wave
        ow[wave * dh + lane] = o;
        if (lane == 0) {
          ow[kSC * dh + wave] = mw;
          ow[kSC * dh + kSC + wave] = lw;
        }
        CBAR();
        if (wave == 0) {
          float M = -INFINITY;
#pragma unroll
          for (int i = 0; i < kSC; ++i) M = fmaxf(M, ow[kSC * dh + i]);
          float Ls = 0.f, O = 0.f;
#pragma unroll
          for (int i = 0; i < kSC; ++i) {
            const float mi = ow[kSC * dh + i];
            const float f = mi == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mi - M);
            Ls = fmaf(ow[kSC * dh + kSC + i], f, Ls);
            O = fmaf(ow[i * dh + lane], f, O);
          }
          uint64_t* out = a.pb + (int64_t)par * kSRP * a.sp + ((int64_t)bc * H + bh) * kPPart;
          if (lane == 0) {
            ll_put(out, M, E + 1u);
            ll_put(out + 1, Ls, E + 1u);
          }
          ll_put(out + 2 + lane, O, E + 1u);
        }
        CBAR();  // s_big is reused after it
        continue;
      }
      Segs s{nullptr, nullptr, 0, 0, 0u, 0u, 30, 0};
      float* dst = s_big;
      if (ph == PH_A || ph == PH_HEAD) {
        if (l > 0) s = Segs{xq, xq, kSQ * D, 0, E - 4u, 0u, 30, 0};
      } else if (ph == PH_C) {
        // the partials of every (chunk, head), then rows uc*16 .. +16 of the four x quarters
        s = Segs{a.pb + (int64_t)par * kSRP * a.sp, xq + uc * 16, np, l > 0 ? 4 * 16 : 0, E + 1u, E - 4u, 4, D};
      } else if (ph == PH_D) {
        s = Segs{a.mb + ((int64_t)par * kSRM + rm) * a.sm, xq, D, 0, E + 2u, 0u, 30, 0};
        dst = s_xmid;
      } else {  // PH_E
        s = Segs{a.hb + ((int64_t)par * kSRH + rh) * a.sh + qE * KQ, xq, KQ, 0, E + 3u, 0u, 30, 0};
      }
      const int n = s.n0 + s.n1;
      if (n) presleep(t_in, prev);
      bool first = true;  // this thread's words of the first pass were all there at its first poll
      for (int b0 = 0; b0 < n; b0 += kSC * 64 * kGW) {  // collective read, kGW words per thread per pass
        const uint64_t* src[kGW];
        uint64_t wv[kGW];
        bool have[kGW], seg1[kGW];
#pragma unroll
        for (int j = 0; j < kGW; ++j) {
          const int i = b0 + tid + kSC * 64 * j, i1 = i - s.n0;
          have[j] = i >= n;
          seg1[j] = i1 >= 0;
          src[j] = have[j] ? s.p0 : seg1[j] ? s.p1 + (int64_t)(i1 >> s.sh1) * s.st1 + (i1 & ((1 << s.sh1) - 1)) : s.p0 + i;
        }
        bool all = false;
        for (int spins = 0; spins < kPSpin; ++spins) {
#pragma unroll
          for (int j = 0; j < kGW; ++j) {
            if (!have[j]) {
              wv[j] = __hip_atomic_load(src[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              have[j] = (uint32_t)(wv[j] >> 32) == (seg1[j] ? s.e1 : s.e0);
            }
          }
          all = true;
#pragma unroll
          for (int j = 0; j < kGW; ++j) all = all && have[j];
          if (all) break;
          if (b0 == 0) first = false;
          if ((spins & 255) == 255 && (lds_load(&s_sh.fail) ||
                                       __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0))
            break;
          if (spins < 8)
            __builtin_amdgcn_s_sleep(1);
          else
            __builtin_amdgcn_s_sleep(4);
        }
#pragma unroll
        for (int j = 0; j < kGW; ++j) {
          const int idx = b0 + tid + kSC * 64 * j;
          if (idx < n) dst[idx] = __uint_as_float((uint32_t)wv[j]);
        }
        if (!all) give_up(a.err);
        CBAR();
      }
      if (n) {
        const uint32_t nxt = next_sleep(t_in, prev, __all(first));
        if (lane == 0) s_wait[wave * 8 + ph] = nxt;
      }
      // ---- the vector whose digit planes the units read ----
      int K = D;
      const float* vsrc = s_xin;
      if (ph == PH_A || ph == PH_HEAD) {
        for (int i = tid; i < D; i += kSC * 64)
          s_xin[i] = l == 0 ? a.x[i] : (s_big[i] + s_big[D + i]) + (s_big[2 * D + i] + s_big[3 * D + i]);
      } else if (ph == PH_C) {
        // the unit's x rows; per head M = max m_c, den = sum l_c 2^(m_c - M); chunk weights 2^(m_c - M) / den
        if (tid < 16) {
          const float* xw = s_big + np;
          s_xin[uc * 16 + tid] = l == 0 ? a.x[uc * 16 + tid] : (xw[tid] + xw[16 + tid]) + (xw[32 + tid] + xw[48 + tid]);
        }
        float* cw = s_big + np + 64;
        if (tid < nact * H) {
          const int hh = tid % H;
          float M = -INFINITY;
          for (int cc = 0; cc < nact; ++cc) M = fmaxf(M, s_big[(cc * H + hh) * kPPart]);
          float den = 0.f;
          for (int cc = 0; cc < nact; ++cc)
            den = fmaf(s_big[(cc * H + hh) * kPPart + 1], __builtin_amdgcn_exp2f(s_big[(cc * H + hh) * kPPart] - M),
                       den);
          cw[tid] = __builtin_amdgcn_exp2f(s_big[tid * kPPart] - M) / den;
        }
        CBAR();
        for (int i = tid; i < H * dh; i += kSC * 64) {
          const int hh = i / dh, d = i % dh;
          float att = 0.f;
          for (int cc = 0; cc < nact; ++cc) att = fmaf(s_big[(cc * H + hh) * kPPart + 2 + d], cw[cc * H + hh], att);
          s_xmid[i] = att;
        }
        vsrc = s_xmid;
      } else if (ph == PH_D) {
        vsrc = s_xmid;
      } else {  // PH_E: the h quarter
        vsrc = s_big;
        K = KQ;
      }
      CBAR();
      // ---- digit planes: X = rint(v 2^(27 - E)), four signed base-128 digits (thread t: elements 4t .. 4t+3) ----
      float unit, ssum;
      {
        const bool live = tid < K / 4;
        float4 v = live ? reinterpret_cast<const float4*>(vsrc)[tid] : make_float4(0.f, 0.f, 0.f, 0.f);
        float s2 = v.x * v.x;
        s2 = fmaf(v.y, v.y, s2);
        s2 = fmaf(v.z, v.z, s2);
        s2 = fmaf(v.w, v.w, s2);
        v = make_float4(v.x * wq.x, v.y * wq.y, v.z * wq.z, v.w * wq.w);
        float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        s2 = wave_sum_dpp(s2);
        mx = wave_max_dpp(mx);
        if (lane == 0) {
          s_red[2 * wave] = s2;
          s_red[2 * wave + 1] = mx;
        }
        CBAR();
        float tot = 0.f, m = 0.f;
#pragma unroll
        for (int i = 0; i < kSC; ++i) {
          tot += s_red[2 * i];
          m = fmaxf(m, s_red[2 * i + 1]);
        }
        int Ex = 0;
        if (m > 0.f) (void)frexpf(m, &Ex);  // m = f 2^Ex, f in [0.5, 1): every |v| < 2^Ex
        Ex = max(Ex, -96);                  // 2^(27 - Ex) stays finite; smaller vectors lose their low bits only
        const float up = ldexpf(1.0f, 27 - Ex);
        if (live) {
          const float vv[4] = {v.x, v.y, v.z, v.w};
          uint32_t pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            int X = __float2int_rn(vv[i] * up);  // |X| < 2^27
#pragma unroll
            for (int p = 0; p < 3; ++p) {
              const int d = ((X + 64) & 127) - 64;
              pk[p] |= (uint32_t)(d & 0xFF) << (8 * i);
              X = (X - d) >> 7;
            }
            pk[3] |= (uint32_t)(X & 0xFF) << (8 * i);  // |X| <= 64 here
          }
#pragma unroll
          for (int p = 0; p < 4; ++p) reinterpret_cast<uint32_t*>(s_pln + p * kSPlane)[tid] = pk[p];
        }
        unit = ldexpf(1.0f, Ex - 27);
        ssum = tot;
        CBAR();
      }
      const float inv = 1.0f / sqrtf(ssum / (float)D + a.eps);  // RMSNorm phases (A, D, head)
      if (wave >= nunits) continue;
      // ---- this wave's unit: its tiles, one or two groups (gate and up) of 16 row values ----
      int t0, ntile, soff, ngrp = 1;
      uint32_t lb = lbase, pb0 = pbase;
      if (ph == PH_A) {
        t0 = 0;
        ntile = KB;
        soff = sb;
      } else if (ph == PH_C) {
        t0 = tC0;
        ntile = KB;
        soff = sb + sC;
      } else if (ph == PH_D) {
        t0 = tD0 + wave * 2 * KB;
        ntile = KB;
        ngrp = 2;
        soff = sb + sD + wave * unit_scale_bytes(g, U_D);
      } else if (ph == PH_E) {
        t0 = tE0 + wave * g.KBQ;
        ntile = g.KBQ;
        soff = sb + sE + wave * unit_scale_bytes(g, U_E);
      } else {
        t0 = wave * KB;
        ntile = KB;
        lb = (uint32_t)L * per + (uint32_t)shd;
        pb0 = (uint32_t)L * (uint32_t)nl;
        soff = (L % kSSb) * kSSbBytes + wave * unit_scale_bytes(g, U_H);
      }
      if (!wait_loaded(lb + t0 + ngrp * ntile - 1, a.err)) return;
      float vals[2] = {0.f, 0.f};
      {
        const int i = lane & 15, grp = lane >> 4;
        // lanes of MFMA rows 0..3 read plane i; rows 4..15 read zeros: one address select, no branch
        const int8_t* abase = i < 4 ? s_pln + i * kSPlane + grp * 16 : s_zero;
        const int astep = i < 4 ? 64 : 0;
        for (int gi = 0; gi < ngrp; ++gi) {
          const uint8_t* sc = s_sbuf + soff + gi * (B64 ? ntile * 16 * 2 : 64);
          uint32_t slot = __builtin_amdgcn_readfirstlane((pb0 + t0 + gi * ntile) % kSRing);
          int kb = 0;
          i32x4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
          double acc = 0.0;
          for (int t = 0; t < ntile; t += 4) {
            i32x4 av[4], bv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {  // tiles past ntile read valid LDS and are not used
              av[u] = *reinterpret_cast<const i32x4*>(abase + min(kb + u, ntile - 1) * astep);
              const uint32_t su = slot + u >= kSRing ? slot + u - kSRing : slot + u;
              bv[u] = *reinterpret_cast<const i32x4*>(s_ring + su * 1024 + lane * 16);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              if (t + u < ntile) {  // uniform
                if constexpr (!B64) {
                  if (u & 1)
                    c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u], bv[u], c1, 0, 0, 0);
                  else
                    c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u], bv[u], c0, 0, 0, 0);
                } else {
                  const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u], bv[u], i32x4{0, 0, 0, 0}, 0, 0, 0);
                  const double T =
                      (double)c[0] + 128.0 * (double)c[1] + 16384.0 * (double)c[2] + 2097152.0 * (double)c[3];
                  acc = fma(T, (double)__half2float(reinterpret_cast<const __half*>(sc)[(t + u) * 16 + i]), acc);
                }
              }
            }
            slot = slot + 4 >= kSRing ? slot + 4 - kSRing : slot + 4;
            kb += 4;
          }
          if constexpr (!B64) {
            const double T = (double)(c0[0] + c1[0]) + 128.0 * (double)(c0[1] + c1[1]) +
                             16384.0 * (double)(c0[2] + c1[2]) + 2097152.0 * (double)(c0[3] + c1[3]);
            vals[gi] = (float)(T * (double)unit * (double)reinterpret_cast<const float*>(sc)[i]);
          } else {
            vals[gi] = (float)(acc * (double)unit);
          }
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) __hip_atomic_fetch_add(&s_sh.udone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      // ---- the phase's outputs ----
      if (ph == PH_A) {
        const int j = lane & 15;
        const TileSrc ts = tile_src(g, U_A, ua, 0, j);
        const int hd = ts.row / dh, d = ts.row % dh;
        float val = vals[0] * inv + ep0;
        const float partner = __shfl_xor(val, 8, 64);
        if (hd < H + Hk) {  // rotary on q and k: x cos + rotate_half(x) sin (qwen2.py:64-71)
          const float c = ep1, sn = ep2;
          val = j < 8 ? val * c + (-partner) * sn : val * c + partner * sn;
        }
        if (lane < 16) {
          ll_put(a.qkvb + (int64_t)par * R + ts.row, val, E);
          if (hd >= H) {  // k or v head: this token's cache row
            const int kvh = hd - H;
            float* cache = kvh < Hk ? a.k_cache : a.v_cache;
            const int gh = kvh < Hk ? kvh : kvh - Hk;
            cache[(((int64_t)l * Hk + gh) * a.cap + pos) * dh + d] = val;
          }
        }
      } else if (ph == PH_C) {
        if (lane < 16) {
          const int row = uc * 16 + lane;
          const float xm = s_xin[row] + vals[0];
#pragma unroll
          for (int rr = 0; rr < kSRM; ++rr) ll_put(a.mb + ((int64_t)par * kSRM + rr) * a.sm + row, xm, E + 2u);
        }
      } else if (ph == PH_D) {
        if (lane < 16) {
          const float gv = vals[0] * inv, uv = vals[1] * inv;
          const float hv = (gv / (1.0f + expf(-gv))) * uv;
          const int j = (wave == 0 ? ud0 : ud1) * 16 + lane;
#pragma unroll
          for (int rr = 0; rr < kSRH; ++rr) ll_put(a.hb + ((int64_t)par * kSRH + rr) * a.sh + j, hv, E + 3u);
        }
      } else if (ph == PH_E) {
        if (lane < 16) {
          const int row = ((wave == 0 ? ue0 : ue1) / kSQ) * 16 + lane;
          const float y = qE == 0 ? s_xmid[row] + vals[0] : vals[0];
#pragma unroll
          for (int rr = 0; rr < kSRX; ++rr) ll_put(a.xb + ((int64_t)par * kSRX + rr) * a.sx + qE * D + row, y, E + 4u);
        }
      } else {  // PH_HEAD: logits, and this wave's best row (larger value, then the lower row)
        const int row = (wave == 0 ? uh0 : uh1) * 16 + (lane & 15);
        float best = -INFINITY;
        int bidx = 0x7fffffff;
        if (lane < 16 && row < g.V) {
          const float lg = vals[0] * inv + ep0;
          a.logits[row] = lg;
          best = lg;
          bidx = row;
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          const float ob = __shfl_xor(best, o, 64);
          const int oi = __shfl_xor(bidx, o, 64);
          if (ob > best || (ob == best && oi < bidx)) {
            best = ob;
            bidx = oi;
          }
        }
        if (lane == 0) {
          s_hbv[wave] = best;
          s_hbi[wave] = bidx;
        }
      }
    }
  }

  // ---- the greedy pick ----
  if (tid < 64 * kSC && (tid >> 6) >= nhu && lane == 0) {
    s_hbv[tid >> 6] = -INFINITY;
    s_hbi[tid >> 6] = 0x7fffffff;
  }
  CBAR();
  if (!a.select) return;
  const uint32_t EH = ebase + (uint32_t)L * 8u;
  if (tid == 0) {
    float b = s_hbv[0];
    int bi = s_hbi[0];
    for (int k = 1; k < kSC; ++k)
      if (s_hbv[k] > b || (s_hbv[k] == b && s_hbi[k] < bi)) {
        b = s_hbv[k];
        bi = s_hbi[k];
      }
    ll_put(a.arg + 2 * w, b, EH);
    ll_put(a.arg + 2 * w + 1, __int_as_float(bi), EH);
  }
  if (w != 0) return;
  {
    const int n = 2 * g.G;  // at most 512: one word per thread
    uint64_t wv = 0;
    bool have = tid >= n;
    for (int spins = 0; spins < kPSpin && !have; ++spins) {
      wv = __hip_atomic_load(a.arg + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      have = (uint32_t)(wv >> 32) == EH;
      if (!have && (spins & 255) == 255 && __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)
        break;
      if (!have) __builtin_amdgcn_s_sleep(1);
    }
    if (tid < n) s_big[tid] = __uint_as_float((uint32_t)wv);
    if (!have) give_up(a.err);
    CBAR();
  }
  uint64_t k = 0;
  for (int i = tid; i < g.G; i += kSC * 64)
    k = max(k, ((uint64_t)ord_bits(s_big[2 * i]) << 32) | (0xffffffffu - (uint32_t)__float_as_int(s_big[2 * i + 1])));
  k = wave_max_u64(k);
  if (lane == 0) s_hbk[wave] = k;
  CBAR();
  uint64_t kb = s_hbk[0];
#pragma unroll
  for (int i = 1; i < kSC; ++i) kb = max(kb, s_hbk[i]);
  int bi = (int)(0xffffffffu - (uint32_t)kb);
  if (bi < 0 || bi >= g.V) bi = 0;  // all-NaN logits: keep a valid row
  const int64_t id = bi;
  for (int64_t cc = tid; cc < a.emb.k; cc += kSC * 64)
    a.x[cc] = (float)a.emb.q[id * a.emb.kp + cc] * sc_at(a.emb, id, cc);
  if (tid == 0) {
    a.history[pos + 1] = id;
    *a.token = id;
    *a.pos = pos + 1;
  }
}

// ---------------------------------------------------------------------------
// Host side: geometry, plan, sizes.
// ---------------------------------------------------------------------------
int64_t replica_words(int64_t n) { return (n + 511) / 512 * 512 + 64; }

int make_geo(const cv3_qwen2_model* m, int G, SGeo* g) {
  CV3_REQUIRE(m, CV3_EINVAL, "null model");
  const int64_t H = m->heads, Hk = m->kv_heads, dh = m->head_dim, D = m->hidden, I = m->inter;
  CV3_REQUIRE(H > 0 && Hk > 0 && H % Hk == 0 && H / Hk <= 8 && dh == 64 && H * dh == D, CV3_EUNSUPPORTED,
              "streamed step: heads %lld / kv heads %lld / head dim %lld", (long long)H, (long long)Hk,
              (long long)dh);
  CV3_REQUIRE(D % 64 == 0 && D <= 1024 && I % (64 * kSQ) == 0 && I / kSQ <= kSPlane, CV3_EUNSUPPORTED,
              "streamed step: hidden %lld must be a multiple of 64 (at most 1024), inter %lld of %d (at most %d)",
              (long long)D, (long long)I, 64 * kSQ, kSQ * kSPlane);
  CV3_REQUIRE(m->layers > 0 && m->layers * 8 + 8 <= 256, CV3_EUNSUPPORTED, "streamed step: %lld layers (at most 31)",
              (long long)m->layers);
  int rc;
  if ((rc = check_qw(m->qkv, "qkv", D))) return rc;
  if ((rc = check_qw(m->o, "o_proj", D))) return rc;
  if ((rc = check_qw(m->gate_up, "gate_up", D))) return rc;
  if ((rc = check_qw(m->down, "down", I))) return rc;
  if ((rc = check_qw(m->head, "llm_decoder", D))) return rc;
  if ((rc = check_qw(m->embedding, "speech_embedding", D))) return rc;
  const cv3_qweight* ws[5] = {&m->qkv, &m->o, &m->gate_up, &m->down, &m->head};
  const bool b64 = m->qkv.block == 64 && m->qkv.kp != 64;
  for (const cv3_qweight* x : ws) {
    CV3_REQUIRE(x->kind == CV3_KIND_Q8, CV3_EUNSUPPORTED, "streamed step: int8 weights only");
    CV3_REQUIRE(x->kp == x->k, CV3_EUNSUPPORTED, "streamed step: K must not be padded");
    const bool xb64 = x->block == 64 && x->kp != 64;
    CV3_REQUIRE(xb64 == b64 && (b64 ? x->scale_dtype == CV3_F16 : x->block == x->kp), CV3_EUNSUPPORTED,
                "streamed step: every matrix per-row scaled (block = K), or every one block 64 with float16 scales");
  }
  CV3_REQUIRE(m->embedding.kind == CV3_KIND_Q8, CV3_EUNSUPPORTED, "streamed step: speech_embedding must be q8");
  CV3_REQUIRE(m->qkv.rows == (H + 2 * Hk) * dh && m->o.rows == D && m->gate_up.rows == 2 * I && m->down.rows == D &&
                  m->embedding.rows >= m->head.rows,
              CV3_EINVAL, "stacked weight rows do not match the geometry");
  SGeo r{};
  r.L = (int)m->layers;
  r.D = (int)D;
  r.H = (int)H;
  r.Hk = (int)Hk;
  r.dh = (int)dh;
  r.I = (int)I;
  r.V = (int)m->head.rows;
  r.G = G;
  r.KB = (int)(D / 64);
  r.KBQ = (int)(I / 64 / kSQ);
  r.R = (int)((H + 2 * Hk) * dh);
  r.nA = r.R / 16;
  r.nC = r.D / 16;
  r.nD = r.I / 16;
  r.nE = (r.D / 16) * kSQ;
  r.nHd = (r.V + 15) / 16;
  r.b64 = b64 ? 1 : 0;
  r.Bbase = G - r.H * kPChunks;
  CV3_REQUIRE(G > 0 && r.Bbase >= r.nA + r.nC && r.nD >= G && 2 * G >= r.nD && 2 * G >= r.nE && 2 * G >= r.nHd,
              CV3_EUNSUPPORTED,
              "streamed step: %d workgroups cannot hold %d qkv + %d o_proj units and %d attention items, with "
              "every workgroup owning one to two [gate; up] units",
              G, r.nA, r.nC, r.H * kPChunks);
  *g = r;
  return CV3_OK;
}

// Per workgroup: the qkv / o_proj units on fixed workgroups (0 .. nA - 1, then nC), attention items on the
// last H * 8; [gate; up] and down units by longest-processing-time onto the least loaded workgroup (load in
// tiles; two down units of one workgroup share their K quarter, so one h quarter feeds both); head units
// likewise, on their own.
int make_plan(const SGeo& g, std::vector<int64_t>& plan, int64_t* total_bytes) {
  const int G = g.G;
  plan.assign((size_t)G * kSPW, 0);
  auto F = [&](int w, int f) -> int64_t& { return plan[(size_t)w * kSPW + f]; };
  std::vector<int64_t> load(G, 0), hload(G, 0);
  for (int w = 0; w < G; ++w) {
    F(w, P_A) = F(w, P_C) = F(w, P_D0) = F(w, P_D1) = F(w, P_E0) = F(w, P_E1) = F(w, P_H0) = F(w, P_H1) = -1;
  }
  for (int u = 0; u < g.nA; ++u) {
    F(u, P_A) = u;
    load[u] += g.KB;
  }
  for (int u = 0; u < g.nC; ++u) {
    F(g.nA + u, P_C) = u;
    load[g.nA + u] += g.KB;
  }
  auto lightest = [&](const std::vector<int64_t>& ld, auto&& fits) {
    int best = -1;
    for (int w = 0; w < G; ++w)
      if (fits(w) && (best < 0 || ld[w] < ld[best])) best = w;
    return best;
  };
  for (int u = 0; u < g.nD; ++u) {
    const int w = lightest(load, [&](int x) { return F(x, P_ND) < 2; });
    if (w < 0) return fail(CV3_EUNSUPPORTED, "streamed step: no room for [gate; up] unit %d", u);
    F(w, P_D0 + F(w, P_ND)) = u;
    ++F(w, P_ND);
    load[w] += 2 * g.KB;
  }
  for (int q = 0; q < kSQ; ++q)
    for (int rb = 0; rb < g.D / 16; ++rb) {
      const int u = rb * kSQ + q;
      const int w = lightest(load, [&](int x) { return F(x, P_NE) == 0 || (F(x, P_NE) == 1 && F(x, P_E0) % kSQ == q); });
      if (w < 0) return fail(CV3_EUNSUPPORTED, "streamed step: no room for down unit %d", u);
      F(w, P_E0 + F(w, P_NE)) = u;
      ++F(w, P_NE);
      load[w] += g.KBQ;
    }
  for (int u = 0; u < g.nHd; ++u) {
    const int w = lightest(hload, [&](int x) { return F(x, P_NH) < 2; });
    if (w < 0) return fail(CV3_EUNSUPPORTED, "streamed step: no room for head unit %d", u);
    F(w, P_H0 + F(w, P_NH)) = u;
    ++F(w, P_NH);
    hload[w] += g.KB;
  }
  int64_t off = 0;
  for (int w = 0; w < G; ++w) {
    const Units lu = region_units(&F(w, 0), false), hu = region_units(&F(w, 0), true);
    int64_t tl = 0, sl = 0, th = 0, shb = 0;
    for (int i = 0; i < lu.n; ++i) {
      tl += unit_tiles(g, lu.type[i]);
      sl += unit_scale_bytes(g, lu.type[i]);
    }
    for (int i = 0; i < hu.n; ++i) {
      th += unit_tiles(g, hu.type[i]);
      shb += unit_scale_bytes(g, hu.type[i]);
    }
    if (sl > kSSbBytes || shb > kSSbBytes)
      return fail(CV3_EUNSUPPORTED, "streamed step: %lld scale bytes for one workgroup's layer", (long long)sl);
    F(w, P_SB) = sl;
    F(w, P_SBH) = shb;
    F(w, P_NL) = tl;
    F(w, P_NHT) = th;
    F(w, P_SPAD) = (sl + 255) / 256 * 256;
    F(w, P_SPADH) = (shb + 255) / 256 * 256;
    F(w, P_STRIDE) = F(w, P_SPAD) + tl * 1024;
    F(w, P_OFF) = off;
    F(w, P_HOFF) = (int64_t)g.L * F(w, P_STRIDE);
    off += F(w, P_HOFF) + F(w, P_SPADH) + th * 1024;
  }
  *total_bytes = off;
  return CV3_OK;
}

int64_t stream_words(const SGeo& g) {
  return 2 * kSRX * replica_words((int64_t)kSQ * g.D) + 2 * (int64_t)g.R +
         2 * kSRP * replica_words((int64_t)kPChunks * g.H * kPPart) + 2 * kSRM * replica_words(g.D) +
         2 * kSRH * replica_words(g.I) + 2 * (int64_t)g.G;
}

int default_workgroups(int G) {
  if (G > 0) return G;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess)
    return 256;
  return std::min(cus, 256);
}

}  // namespace

extern "C" {

int cv3_qwen2_stream_size(const cv3_qwen2_model* m, int workgroups, int64_t* data_bytes, int64_t* plan_words,
                          int64_t* exchange_words) {
  CV3_ALIVE();
  SGeo g;
  int rc = make_geo(m, default_workgroups(workgroups), &g);
  if (rc) return rc;
  std::vector<int64_t> plan;
  int64_t bytes = 0;
  if ((rc = make_plan(g, plan, &bytes))) return rc;
  if (data_bytes) *data_bytes = bytes;
  if (plan_words) *plan_words = (int64_t)plan.size();
  if (exchange_words) *exchange_words = stream_words(g);
  return CV3_OK;
}

int cv3_qwen2_stream_pack(const cv3_qwen2_model* m, int workgroups, void* data, int64_t data_bytes, int64_t* plan,
                          int64_t plan_words, cv3_stream_t stream) {
  CV3_ALIVE();
  SGeo g;
  int rc = make_geo(m, default_workgroups(workgroups), &g);
  if (rc) return rc;
  std::vector<int64_t> hp;
  int64_t bytes = 0;
  if ((rc = make_plan(g, hp, &bytes))) return rc;
  CV3_REQUIRE(data && plan && data_bytes >= bytes && plan_words >= (int64_t)hp.size(), CV3_EINVAL,
              "stream pack: buffers of %lld bytes and %lld plan words needed", (long long)bytes,
              (long long)hp.size());
  CV3_REQUIRE((uintptr_t)data % 256 == 0, CV3_EINVAL, "stream pack: data must be 256-byte aligned");
  hipStream_t st = stream_of(stream);
  CV3_HIP(hipMemcpyAsync(plan, hp.data(), hp.size() * sizeof(int64_t), hipMemcpyHostToDevice, st));
  PackArgs a{};
  a.g = g;
  const cv3_qweight* ws[5] = {&m->qkv, &m->o, &m->gate_up, &m->down, &m->head};
  for (int i = 0; i < 5; ++i) {
    a.w[i] = reinterpret_cast<const int8_t*>(ws[i]->q);
    a.s[i] = ws[i]->scales;
    a.rows[i] = ws[i]->rows;
    a.kp[i] = ws[i]->kp;
    a.nb[i] = ws[i]->kp / ws[i]->block;
    a.sf16[i] = ws[i]->scale_dtype == CV3_F16;
  }
  a.plan = plan;
  a.out = reinterpret_cast<uint8_t*>(data);
  hipLaunchKernelGGL(k_stream_pack, dim3((unsigned)g.G, (unsigned)(g.L + 1)), dim3(256), 0, st, a);
  CV3_LAUNCHED();
  CV3_HIP(hipStreamSynchronize(st));  // the host plan goes out of scope
  return CV3_OK;
}

int cv3_qwen2_decode_step_stream(const cv3_qwen2_model* m, const cv3_qwen2_state* s, const cv3_qwen2_stream* ws,
                                 const cv3_persist* p, int select, cv3_stream_t stream) {
  CV3_ALIVE();
  CV3_REQUIRE(m && s && ws && p, CV3_EINVAL, "null model, state, weight stream or exchange block");
  SGeo g;
  int rc = make_geo(m, default_workgroups(ws->workgroups), &g);
  if (rc) return rc;
  CV3_REQUIRE(ws->data && ws->plan && ws->workgroups == g.G, CV3_EINVAL,
              "streamed step: the weight stream was packed for %d workgroups, not %d", ws->workgroups, g.G);
  CV3_REQUIRE(s->cap > 0 && s->cap <= (int64_t)kPChunks * kPKeys, CV3_EUNSUPPORTED,
              "streamed step: cache capacity above %d positions", kPChunks * kPKeys);
  CV3_REQUIRE(p->words && p->err && p->words_len >= stream_words(g), CV3_EINVAL,
              "streamed step: exchange words missing or too few");
  CV3_REQUIRE(p->epoch_base != 0, CV3_EINVAL, "streamed step: epoch base 0 is the cleared state");
  int dev = 0, cus = 0, per_cu = 0;
  CV3_HIP(hipGetDevice(&dev));
  CV3_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const void* fn = g.b64 ? (const void*)k_dec_stream<true> : (const void*)k_dec_stream<false>;
  CV3_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kST, 0));
  CV3_REQUIRE(g.G <= per_cu * cus, CV3_EUNSUPPORTED, "streamed step: %d workgroups, %d can be resident", g.G,
              per_cu * cus);
  SArgs a{};
  a.packed = reinterpret_cast<const uint8_t*>(ws->data);
  a.plan = ws->plan;
  a.g = g;
  a.ln1 = m->ln1;
  a.ln2 = m->ln2;
  a.norm = m->norm;
  a.qkv_bias = m->qkv_bias;
  a.head_bias = m->head_bias;
  a.rope_cos = m->rope_cos;
  a.rope_sin = m->rope_sin;
  a.emb = make_qw(m->embedding);
  a.eps = m->eps;
  a.scale = 1.0f / sqrtf((float)g.dh);
  a.k_cache = s->k_cache;
  a.v_cache = s->v_cache;
  a.cap = s->cap;
  a.pos = s->pos;
  a.token = s->token;
  a.history = s->history;
  a.x = s->x;
  a.logits = s->logits;
  a.sx = replica_words((int64_t)kSQ * g.D);
  a.sp = replica_words((int64_t)kPChunks * g.H * kPPart);
  a.sm = replica_words(g.D);
  a.sh = replica_words(g.I);
  uint64_t* wds = p->words;
  a.xb = wds;
  a.qkvb = a.xb + 2 * kSRX * a.sx;
  a.pb = a.qkvb + 2 * (int64_t)g.R;
  a.mb = a.pb + 2 * kSRP * a.sp;
  a.hb = a.mb + 2 * kSRM * a.sm;
  a.arg = a.hb + 2 * kSRH * a.sh;
  a.err = p->err;
  a.epoch_base = p->epoch_base;
  a.select = select ? 1 : 0;
  if (p->cooperative) {
    void* args[] = {&a};
    CV3_HIP(hipLaunchCooperativeKernel(fn, dim3((unsigned)g.G), dim3(kST), args, 0, stream_of(stream)));
  } else {
    if (g.b64)
      hipLaunchKernelGGL((k_dec_stream<true>), dim3((unsigned)g.G), dim3(kST), 0, stream_of(stream), a);
    else
      hipLaunchKernelGGL((k_dec_stream<false>), dim3((unsigned)g.G), dim3(kST), 0, stream_of(stream), a);
    CV3_LAUNCHED();
  }
  return CV3_OK;
}

}  // extern "C"
