// Inclusive prefix sum for gfx950: single-pass decoupled look-back.
//
// Symbols and memref arguments follow the reference's two templates
// (lib/dsl/kernels/scan.cpp): `scan` (x, y, y_lo [n]; totals_hi,
// totals_lo [T = ceil(n/256)], 25 parameters) and `scan_totals` (totals_hi,
// totals_lo, off_hi, off_lo, off_lo2 [T]; y, y_lo [n], 35 parameters). The
// reference needs both launches: a per-256 double-float Blelloch pass, then
// ONE workgroup that serially builds the exact prefix of all T totals
// (scan.cpp:400-452). Here `scan` alone produces the final y in one pass over
// HBM (read x once, write y once: 8 B/element), launched by itself on
// whatever the totals buffers hold:
//
//   * A workgroup of W threads (256..1024, a multiple of 64) has W/64 - 1
//     data waves and one control wave. The data waves own a tile of
//     P (W - 64) elements (P = KH_SCAN_PER_THREAD consecutive per thread,
//     dwordx4 loads); the control wave does the look-back.
//   * When the grid has a workgroup for every tile (one round), tile i is
//     the workgroup of flat index i: its loads go out at kernel entry, the
//     reduction overlaps the session read, and the look-back follows the
//     aggregate's publication at once (scan_one_tile).
//   * Otherwise tiles are handed out in order by an atomic ticket, so a
//     tile only ever waits on tiles already owned by running workgroups
//     (deadlock-free under any grid size). Workgroups are persistent and
//     pipelined: the data waves issue the next tile's loads before the
//     current tile's look-back, and tickets run two ahead, so load, ticket
//     and look-back latencies overlap. Control and data waves run loops of
//     their own, so that each waits only for its own memory operations.
//   * Partial sums are carried in fp64. Every fp32 input is exact in fp64
//     and, for inputs on a common 2^-e grid whose total needs <= 53 bits
//     (every configuration the reference tests: U[0,1) on 2^-24 or
//     mt19937*2^-32 grids up to n = 2^26), every partial sum is EXACT, so
//     y[i] = fl32(exact prefix): the correctly rounded result the reference
//     template computes with double-float + 3-word expansions
//     (scan.cpp:25-38).
//   * Decoupled look-back (Merrill & Garland 2016): each tile publishes its
//     aggregate as soon as it is reduced, then its inclusive prefix. The
//     control wave inspects 64 KH_SCAN_WINDOW predecessors per step (loads
//     issued together) and stops at the nearest inclusive prefix.
//
// Look-back state lives in the caller's totals buffers (the reference ABI
// has no separate workspace) and needs no clearing between calls:
//
//   totals_lo, from its first 8-byte boundary: a 32-byte Header, read by
//   every workgroup at its start,
//       base     low 32 bits: the call's first ticket (ticket base + i is
//                tile i); high 32 bits: the call's generation
//       nonce    device real-time clock when the session began
//       check    mix(base, nonce, header address): the header is recognised
//                only when it matches (and the tickets handed out fit it)
//       failed   bounded waits that ran out (diagnostic; y is NaN there)
//   and 16 B of Counters, updated by every workgroup with atomics, 256 B
//   further on where totals_lo has room (another cache line), else right
//   after the header:
//       counter  32-bit ticket counter, continuing across calls
//       done     workgroups of the current call that have taken their last
//                ticket, and the tickets they took
//   totals_hi, from its first 8-byte boundary: one 16-byte Record per tile
//       0 .. ntiles-2 (the last tile has no successor): {value, check}, the
//       value an fp64 bit pattern. First the tile's aggregate with
//       check = value ^ tag_agg(t), then its inclusive prefix (overwriting
//       it) with check = value ^ tag_inc(t), where t = (generation << 32) |
//       tile and the tags derive from a session key.
//
// A value counts as published only when the record's two words satisfy one
// of those equations for this call's generation and tile. Generations never
// repeat within a session (2^32 calls) and the session key differs per
// header address and per nonce, so stale records of earlier calls, zero- or
// NaN-filled memory and leftovers of other kernels all read as "not yet
// published" (a random 64-bit match is the only way through). A record
// moves as one 16-byte access with the sc1 cache policy (agent scope,
// coherent across the 8 XCD L2s without the L2 write-back/invalidate an
// acquire/release pair would cost on every poll); such an access is not
// guaranteed single-copy atomic, and a torn read simply fails the check and
// is polled again.
//
// Calls that run one after another on the same buffers (stream order) need
// nothing from the host: the last workgroup of a call to count itself done
// moves the first ticket on by the call's tickets (the counter's value),
// adds one to the generation and re-signs the header for the next call. A
// header that is not recognised (fresh, zeroed, garbage, or with a counter
// another kernel wrote) is claimed by one workgroup with a compare-and-swap;
// it starts a new session (first ticket := counter, nonce := the real-time
// clock) while the others wait for the signature. Tickets taken before that
// point are told apart and taken again. Two calls that overlap in time on
// the same totals buffers race (as with any shared output buffer); calls on
// different buffers are independent.
//
// Capacity: 48 B (+4 for alignment) of totals_lo and 16 B per tile but one
// (+4) of totals_hi, both with unit stride; the reference's T = ceil(n/256)
// floats always suffice (a tile is at least 3072 elements, 48 B of T).
// Anything else is refused by writing NaN to y without touching the totals.
//
// Every wait is bounded (KH_SCAN_SPIN_LIMIT polls), so a corrupted state can
// never hang the device:
//   * a look-back that runs out poisons its tile's result (and so every
//     later tile's) with NaN and counts the failure in the header; the call
//     still closes, so the next call runs under a new generation;
//   * a claim left unsigned for the limit (a header that held a claim mark
//     when the call began) is taken over by one of the waiting workgroups,
//     so such a header costs one wait and no failure;
//   * a workgroup whose claims keep stalling (8 limits in all, which needs
//     claimant waves stalled for seconds) counts the failure, writes NaN
//     to its share of y and leaves the header unrecognisable: the call
//     will not close, and the next call then claims a new session rather
//     than reuse this one's generation and records. (Only a claimant that
//     resumes after that and signs escapes this; its call's records could
//     then pass for the next call's.)
// After a call, failed > 0 means y is not to be trusted (NaN, or left as it
// was where a lost ticket's tile was never reached). A claim resets the
// count, so a call in which another workgroup claimed the header after a
// failure shows the failure only as NaN in y.
#include "kh_device.h"
#include "kh_tiles.h"

namespace {

constexpr int kMaxThreads = KH_SCAN_THREADS;
constexpr int kMinThreads = 256;
constexpr int kPerThread = KH_SCAN_PER_THREAD;
#ifndef KH_SCAN_WINDOW
#define KH_SCAN_WINDOW 2
#endif
constexpr int kWindow = KH_SCAN_WINDOW;  // predecessors polled per lane per look-back step
// Polls before a bounded wait gives up (about 1-2 us each: seconds in all).
// A test build sets a small limit to exercise the give-up paths.
#ifndef KH_SCAN_SPIN_LIMIT
#define KH_SCAN_SPIN_LIMIT (1u << 22)
#endif
constexpr uint32_t kSpinLimit = KH_SCAN_SPIN_LIMIT;
constexpr uint64_t kEmpty = ~0ull;

// The header proper, read by every workgroup at its start, and the two
// words every workgroup updates with atomics (Counters). Where totals_lo has
// room, Counters sit 256 B past the header, in another cache line, so the
// header loads do not queue behind the ticket atomics; otherwise right
// after it.
struct Header {
  uint64_t base;  // low 32 bits: the call's first ticket; high 32: its generation
  uint64_t nonce, check;
  uint32_t failed, pad;
};
struct Counters {
  uint32_t counter, pad;  // tickets, mod 2^32 (a call takes far fewer); pad takes
                          // the carries of 64-bit ticket adds and is never read
  uint64_t done;          // low 32 bits: workgroups done; high 32: their tickets
};
static_assert(sizeof(Header) == 32 && sizeof(Counters) == 16, "header layout");
constexpr int64_t kCountersApart = 256;  // bytes from the header, when there is room

__device__ __forceinline__ Counters *counters_of(Header *h, int64_t bytes) {
  char *p = reinterpret_cast<char *>(h);
  return reinterpret_cast<Counters *>(p + (bytes >= kCountersApart + (int64_t)sizeof(Counters)
                                               ? kCountersApart
                                               : (int64_t)sizeof(Header)));
}

struct Record {
  uint64_t value, check;
};
static_assert(sizeof(Record) == 16, "record layout");

// Stafford's mix13 finaliser of SplitMix64: a bijection of 64-bit words.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t nonzero(uint64_t v) { return v == 0 ? 1 : v; }

__device__ __forceinline__ uint64_t session_key(const Header *h, uint64_t nonce) {
  return mix64(reinterpret_cast<uintptr_t>(h) ^ mix64(nonce ^ 0x5ca11ab1e5ca4a11ull));
}

__device__ __forceinline__ uint64_t header_check(const Header *h, uint64_t base, uint64_t nonce) {
  return nonzero(mix64(session_key(h, nonce) ^ mix64(base ^ 0x0c0ffee0ddba11ull)));
}

// Claim marks: the check word of a header being claimed, 256 values that
// differ only in their low byte (the claim's epoch). Never a header's check
// word but by a random coincidence (2^-56).
__device__ __forceinline__ uint64_t claim_mark(const Header *h) {
  return mix64(reinterpret_cast<uintptr_t>(h) ^ 0xc1a1bedc1a1bedull) & ~0xffull;
}
__device__ __forceinline__ bool is_claim_mark(const Header *h, uint64_t v) { return (v & ~0xffull) == claim_mark(h); }

// Record tags of tile i of the call with generation g: a session key XOR
// t = (g << 32) | i, one key per kind of value. A record holds the tile's
// aggregate with check = value ^ agg_tag, and later its inclusive prefix
// (overwriting it) with check = value ^ inc_tag. Within a session (the
// generation counts its calls), distinct t give distinct tags; the two kinds use unrelated keys, and a record written under another
// session (or never written) passes only if its words happen to XOR to a
// value fixed by unrelated mix64 outputs. A read torn between the two words
// of one publication passes only when both values are equal (and then it
// reads that value correctly).
struct Keys {
  uint64_t agg, inc;
};

__device__ __forceinline__ Keys record_keys(uint64_t key) { return Keys{key, mix64(key ^ 0x1dc0ffee5eedull)}; }

__device__ __forceinline__ uint64_t tag(uint64_t key, uint64_t t) { return key ^ t; }

template <typename T>
__device__ __forceinline__ T ld(const T *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ void st(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ T fetch_add(T *p, T v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t bits(double v) { return (uint64_t)__double_as_longlong(v); }

// Records move as one 16-byte buffer access each, with the sc1 cache policy
// (agent scope, coherent across the XCDs' L2s: the bits relaxed agent-scope
// atomics carry). Such an access is not guaranteed to be single-copy atomic;
// a torn one fails the check and is polled again.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kSc1 = 16;  // cache-policy operand of the buffer builtins: sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t record_rsrc(const Record *r) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<Record *>(r), (short)0, 0x7fffffff, 0x00020000);
}

// Publishes one value of tile `tile` when `on`, from lane 0: its aggregate
// (key keys.agg) or its inclusive prefix (key keys.inc, replacing the
// aggregate); t is the tile's tag input. (One store from the whole wave, its
// other lanes addressing past the resource's range, keeps the compiler's
// wait counts exact on every path, but measured slower: 117 against 103 us
// for the scan at n = 2^26.)
__device__ __forceinline__ void publish(Record *rec, bool on, int64_t tile, uint64_t key, uint64_t t, double v,
                                        int lane) {
  const uint64_t b = bits(v), c = b ^ tag(key, t);
  const u32x4 w = {(unsigned)b, (unsigned)(b >> 32), (unsigned)c, (unsigned)(c >> 32)};
  if (on && lane == 0)
    __builtin_amdgcn_raw_buffer_store_b128(w, record_rsrc(rec), (uint32_t)tile * (uint32_t)sizeof(Record), 0, kSc1);
}

// The call's view of the state: where it is, the ticket of tile 0 (low 32
// bits of `base`) and the generation (high 32), and the session keys the
// record tags derive from.
struct Session {
  Header *h;
  Counters *c;
  Record *rec;
  uint64_t base;
  Keys keys;
};

__device__ __forceinline__ uint32_t first_ticket(uint64_t base) { return (uint32_t)base; }
// Tag input of tile i: (generation << 32) | i.
__device__ __forceinline__ uint64_t tag_of(uint64_t base, int64_t tile) {
  return (base & 0xffffffff00000000ull) | (uint32_t)tile;
}

// Run by one thread per workgroup at the start of a multi-tile call. Takes
// the session and the workgroup's first `take` tickets: two (t0 < t1, both
// >= base), one (t0; t1 stands for "no second tile" and equals t0), or none
// when tiles go by workgroup index; false if the header could not be
// established within the bounded wait. The header loads and the ticket
// atomics go out together, so a recognised header costs one round trip.
struct Opened {
  uint64_t base, nonce;
  uint32_t t0, t1;
  bool ok;
};

// Takes the workgroup's starting tickets again (one atomic), keeping a
// second ticket already at or past the session's first: the tickets taken
// before a session began are not tiles of its call.
__device__ __forceinline__ void retake_tickets(Opened &o, Counters *c, uint32_t take) {
  if (take == 0) return;
  if ((int32_t)(o.t1 - first_ticket(o.base)) < 0) {
    o.t0 = fetch_add(&c->counter, take);
    o.t1 = o.t0 + (take - 1);
  } else if ((int32_t)(o.t0 - first_ticket(o.base)) < 0) {
    o.t0 = o.t1;
    o.t1 = fetch_add(&c->counter, 1u);
  }
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t x, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)x, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

// Run by the whole control wave; the result is lane 0's.
__device__ __forceinline__ Opened open_session(Header *h, Counters *c, int64_t ntiles, uint64_t nblocks,
                                               uint32_t take, int lane) {
  Opened o;
  o.ok = true;
  // base, nonce and check in one load instruction of lanes 0-2: one request
  // per workgroup to the header's line (every workgroup reads that line,
  // and the requests for one line queue where it lives: three loads each
  // took 2.4 us to come back for 89 workgroups at n = 10^6).
  uint64_t word = 0;
  if (lane < 3) word = ld(reinterpret_cast<const uint64_t *>(h) + lane);
  // A pair is two consecutive tickets from one atomic: the workgroups'
  // start-up atomics on the counter serialise, one per workgroup instead of
  // two.
  o.t0 = o.t1 = 0;
  if (take != 0 && lane == 0) {
    o.t0 = fetch_add(&c->counter, take);
    o.t1 = o.t0 + (take - 1);
  }
  o.base = readlane_u64(word, 0);
  o.nonce = readlane_u64(word, 1);
  const uint64_t seen0 = readlane_u64(word, 2);
  if (lane != 0) return o;
  // A call takes every ticket below ntiles once and at most two more per
  // workgroup, all >= base: a ticket outside that range means the counter
  // was changed behind the header's back (another kernel wrote it), and the
  // header is not taken as valid even though its check matches. (Without
  // tickets there is nothing to check.)
  const uint64_t span = (uint64_t)ntiles + 2ull * nblocks + 4;
  auto in_range = [&]() { return take == 0 || (uint32_t)(o.t1 - first_ticket(o.base)) < span; };
  bool signed0 = seen0 == header_check(h, o.base, o.nonce);
  // Valid: the header is stable for the whole call (only the last workgroup
  // to finish changes it), so the three words belong together.
  if (signed0 && in_range()) return o;
  if (signed0 && take != 0 && (int32_t)(o.t1 - first_ticket(o.base)) < 0) {
    // Signed, but the tickets precede the session's first ticket. The header
    // loads and the ticket atomic are relaxed and complete in either order,
    // so this is what a workgroup sees when another workgroup of this call
    // claimed the header after this one's atomic and signed it before its
    // loads: the session is open and only the tickets predate it. Take them
    // again; the acquire fence orders everything that follows after the
    // claimant's writes (the signature read above is its release store).
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    retake_tickets(o, c, take);
    if (in_range()) return o;
    // Still outside: the counter itself was moved back. Claim afresh.
  }
  // Not recognised (or read while a claimant was writing it). `check` is
  // read with acquire ordering before base and nonce: when it is a
  // claimant's signature, the base and nonce read after it are the ones it
  // signs. A workgroup claims the header only from a check value that is
  // unsigned (or the signature found with an inconsistent counter), with a
  // compare-and-swap that writes a claim mark, so exactly one claims it; the
  // others wait for the new signature.
  //
  // A claim mark that stays unsigned for kSpinLimit polls (a header that
  // held a mark when the call began: a claim cut short, or a coincidence) is
  // claimed in turn, under the next epoch's mark, by one of the waiting
  // workgroups; every wait counts its polls from the last change of the
  // check word. (A claimant that is alive signs within microseconds: one
  // thread, a handful of stores. Only a claimant wave stalled for seconds
  // could sign after its claim was taken over.)
  const uint64_t mark = claim_mark(h);
  uint64_t last = 0;
  uint32_t spins = 0;
  for (uint32_t polls = 0;; ++polls) {
    const uint64_t seen = __hip_atomic_load(&h->check, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
    o.base = ld(&h->base);
    o.nonce = ld(&h->nonce);
    if (seen == header_check(h, o.base, o.nonce) && !(signed0 && seen == seen0)) break;
    if (seen != last) {
      last = seen;
      spins = 0;
    }
    const bool claimed = is_claim_mark(h, seen);
    if (!claimed || spins > kSpinLimit) {
      uint64_t expect = seen;
      const uint64_t mine = claimed ? mark | ((seen + 1) & 0xff) : mark;
      if (__hip_atomic_compare_exchange_strong(&h->check, &expect, mine, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT)) {
        // A read-modify-write, so every ticket before it precedes the
        // session's first ticket and every ticket after it follows. The
        // generation may start anywhere: the session key carries the nonce.
        o.nonce = __builtin_amdgcn_s_memrealtime();
        o.base = ((uint64_t)(uint32_t)o.nonce << 32) | fetch_add(&c->counter, 0u);
        st(&h->base, o.base);
        st(&h->nonce, o.nonce);
        st(&c->done, uint64_t(0));
        st(&h->failed, 0u);
        __hip_atomic_store(&h->check, header_check(h, o.base, o.nonce), __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      continue;  // another workgroup changed the word first: read it again
    }
    if (polls > 8 * kSpinLimit) {
      // Claims kept stalling: give up. The workgroup's tickets are lost
      // and the call's last workgroup never counts itself done, so this
      // call does not re-sign the header. Leave it unrecognisable (0 is
      // neither a signature nor a claim mark), so that a later call claims
      // a new session, with new record keys, instead of running under this
      // call's generation and taking its records for its own.
      fetch_add(&h->failed, 1u);
      __hip_atomic_store(&h->check, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      o.ok = false;
      return o;
    }
    ++spins;
    __builtin_amdgcn_s_sleep(2);
  }
  retake_tickets(o, c, take);
  return o;
}

// Counts a workgroup as finished with the call's tickets, adding the
// number it took (`tickets`: its first one or two plus one per tile-loop
// step that took one, all >= base). Issued by one thread as soon as the workgroup's
// last ticket has come back (one at or past the last tile).
__device__ __forceinline__ uint64_t count_done(Counters *c, uint32_t tickets) {
  return fetch_add(&c->done, ((uint64_t)tickets << 32) | 1u);
}

// Run when the workgroup ends, with count_done's result. The last workgroup
// of the call to count itself (every ticket of the call has then come back)
// re-signs the header for the next call: its first ticket is this call's
// plus all the tickets of this call (the counter's value), its generation
// one more.
__device__ __forceinline__ void close_session(Header *h, Counters *c, uint64_t base, uint64_t nonce,
                                              uint64_t done_before, uint32_t tickets, uint32_t nblocks) {
  if ((uint32_t)done_before != nblocks - 1) return;
  const uint32_t next_ticket = first_ticket(base) + (uint32_t)(done_before >> 32) + tickets;
  const uint64_t next = ((base & 0xffffffff00000000ull) + (1ull << 32)) | next_ticket;
  st(&c->counter, next_ticket);  // already its value, unless something else wrote it
  st(&h->base, next);
  st(&c->done, uint64_t(0));
  st(&h->check, header_check(h, next, nonce));
}


// DPP move of an fp64 value (two 32-bit halves, same control). Lanes the
// control does not write (row_mask) or that have no source (bound_ctrl) get 0.
template <int CTRL, int ROW_MASK, bool BOUND_CTRL>
__device__ __forceinline__ double dpp_f64(double x) {
  const long long b = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, ROW_MASK, 0xf, BOUND_CTRL);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, ROW_MASK, 0xf, BOUND_CTRL);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// Inclusive scan over the 64 lanes of a wave: Hillis-Steele within each
// 16-lane row (row_shr 1, 2, 4, 8), then row 0's total into row 1 and row
// 2's into row 3 (row_bcast:15), then the first half's total into rows 2
// and 3 (row_bcast:31). gfx9 DPP encodings.
__device__ __forceinline__ double wave_incl_scan_f64(double x) {
  x += dpp_f64<0x111, 0xf, true>(x);
  x += dpp_f64<0x112, 0xf, true>(x);
  x += dpp_f64<0x114, 0xf, true>(x);
  x += dpp_f64<0x118, 0xf, true>(x);
  x += dpp_f64<0x142, 0xa, false>(x);
  x += dpp_f64<0x143, 0xc, false>(x);
  return x;
}

__device__ __forceinline__ double readlane_f64(double x, int lane) {
  const long long b = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_readlane((int)b, lane);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// Sum over the 64 lanes of a wave, the same in every lane: the last lane of
// the DPP scan. (DPP moves are ALU operations; a butterfly of __shfl_xor
// goes through LDS permutes. The look-back and the aggregate are on the
// critical path of every tile: the DPP form measured 12.4 against 12.8 us
// for the scan at n = 10^6, and 102.2-102.8 against 102.9-103.7 us at 2^26.)
__device__ __forceinline__ double wave_sum_f64(double v) { return readlane_f64(wave_incl_scan_f64(v), kh::kWave - 1); }

// A data wave's segment: kRows rows of 256 consecutive elements; lane l
// holds elements [256 k + 4 l, 256 k + 4 l + 4) of row k in v[4k .. 4k+3],
// so each row is one fully coalesced 16-byte access per lane.
//
// Tile data moves through buffer instructions over a resource that spans
// exactly the tile's elements inside [0, n): the hardware range check makes
// loads past n read 0 and drops stores past n. The same instructions are
// issued for every tile, full or partial, with no data-dependent branches
// around them, which keeps the vector-memory wait counts exact (a branch
// with a variable number of memory operations forces waits for all of them).
// VEC (16-byte aligned x and y, n a multiple of 4): dwordx4 accesses, each
// wholly inside or wholly outside the range; otherwise dword accesses.
constexpr int kRows = kPerThread / 4;
static_assert(kPerThread % 4 == 0, "rows of float4");
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor: 32-bit data format

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const float *base, int64_t elems) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, (int)(elems * 4), kRsrcWord3);
}

// The dword path passes `lane` through an empty asm, so that its sixteen
// per-dword offsets are computed where the accesses are issued instead of
// being hoisted out of the tile loop, where they would hold sixteen
// registers for its whole length (a 1024-thread workgroup has 128).
template <bool VEC>
__device__ __forceinline__ void load_seg(float (&v)[kPerThread], __amdgpu_buffer_rsrc_t r, int seg, int lane) {
  if (!VEC) asm volatile("" : "+v"(lane));
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    const int e = seg + 256 * k + 4 * lane;
    if (VEC) {
      const u32x4 f = __builtin_amdgcn_raw_buffer_load_b128(r, 4 * e, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[4 * k + j] = __uint_as_float(f[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[4 * k + j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, 4 * (e + j), 0, 0));
    }
  }
}

template <bool VEC>
__device__ __forceinline__ void store_seg(const float (&o)[kPerThread], __amdgpu_buffer_rsrc_t r, int seg,
                                          int lane) {
  if (!VEC) asm volatile("" : "+v"(lane));
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    const int e = seg + 256 * k + 4 * lane;
    if (VEC) {
      u32x4 f;
#pragma unroll
      for (int j = 0; j < 4; ++j) f[j] = __float_as_uint(o[4 * k + j]);
      __builtin_amdgcn_raw_buffer_store_b128(f, r, 4 * e, 0, 0);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o[4 * k + j]), r, 4 * (e + j), 0, 0);
    }
  }
}

// One look-back window: predecessors end, end-1, ..., end - 64 kWindow + 1;
// lane l, slot j holds distance d = l + 64 j behind `end`. A poll only
// issues the loads of the records' two words; `decode` reads them (waiting
// for the loads there, not at the poll), so the first poll of a look-back
// can be issued before a barrier and land while the workgroup works.
struct Window {
  uint64_t value[kWindow], chk[kWindow];
};

__device__ __forceinline__ void poll_window(Window &w, const Session &s, int64_t end, int lane) {
  // Byte offsets of the records from the (wave-uniform) record base: 32-bit
  // and below 2^31 (tile indices are below 2^27).
#pragma unroll
  for (int j = 0; j < kWindow; ++j) {
    const int64_t idx = end - lane - kh::kWave * j;
    // The empty asm keeps a repeated poll of the same records from being
    // merged with the previous one (the loads are not marked volatile).
    uint32_t off = (uint32_t)(idx >= 0 ? idx : 0) * (uint32_t)sizeof(Record);
    asm volatile("" : "+v"(off));
    const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(record_rsrc(s.rec), off, 0, kSc1);
    w.value[j] = ((uint64_t)q.y << 32) | q.x;
    w.chk[j] = ((uint64_t)q.w << 32) | q.z;
  }
}

// Waits, right here, until a polled window has landed. The look-back's
// polls are needed at once anyway; waiting for them where they are issued
// (not only where they are decoded) leaves no poll in flight on any path of
// the compiler's structured control flow. Such a path (one the look-back
// never takes) would otherwise carry the poll's registers "pending" into the
// next step, where their reuse waits for every memory operation in flight,
// the previous step's record stores included.
__device__ __forceinline__ void settle(const Window &w) {
#pragma unroll
  for (int j = 0; j < kWindow; ++j) asm volatile("" ::"v"(w.value[j]), "v"(w.chk[j]));
}

// Published values of a polled window, kEmpty where unpublished (never an
// fp64 sum of fp32 inputs: those keep the low 29 mantissa bits of every
// operand clear, and fp64 addition yields only canonical or propagated
// NaNs). inc: the inclusive prefix where published; ag: the aggregate where
// only that is. Slots before tile 0 act as an inclusive prefix of value 0.
__device__ __forceinline__ void decode(const Window &w, const Session &s, int64_t end, int lane,
                                       uint64_t (&inc)[kWindow], uint64_t (&ag)[kWindow]) {
#pragma unroll
  for (int j = 0; j < kWindow; ++j) {
    const int64_t idx = end - lane - kh::kWave * j;
    const uint64_t t = tag_of(s.base, idx);
    const bool before = idx < 0;
    const uint64_t x = w.chk[j] ^ w.value[j];
    inc[j] = before ? 0ull : (x == tag(s.keys.inc, t) ? w.value[j] : kEmpty);
    ag[j] = before ? kEmpty : (x == tag(s.keys.agg, t) ? w.value[j] : kEmpty);
  }
}

// Exclusive prefix of `tile` from its predecessors' published records (run
// by one whole wave; the result is wave-uniform), starting from window `w`,
// already polled for end = tile - 1. Records only ever go from unpublished
// to aggregate to inclusive prefix within a call, so an early poll is a
// valid (if possibly incomplete) observation. NaN if the bounded wait ran
// out.
__device__ __forceinline__ double look_back(const Session &s, int64_t tile, int lane, Window w) {
  double excl = 0.0;
  int64_t end = tile - 1;  // newest predecessor still to account for
  uint32_t spins = 0;
  for (;;) {
    uint64_t inc[kWindow], ag[kWindow];
    decode(w, s, end, lane, inc, ag);
    // Nearest inclusive prefix, and whether every nearer predecessor has at
    // least published its aggregate.
    int first = kWindow * kh::kWave;
#pragma unroll
    for (int j = kWindow - 1; j >= 0; --j) {
      const uint64_t m = __ballot(inc[j] != kEmpty);
      if (m) first = kh::kWave * j + __builtin_ctzll(m);
    }
    bool pending = false;
#pragma unroll
    for (int j = 0; j < kWindow; ++j) {
      const int d = lane + kh::kWave * j;
      if (d < first && ag[j] == kEmpty) pending = true;
    }
    if (__ballot(pending) != 0) {
      if (++spins > kSpinLimit) {
        if (lane == 0) fetch_add(&s.h->failed, 1u);
        return __builtin_nan("");
      }
      __builtin_amdgcn_s_sleep(1);
      poll_window(w, s, end, lane);
      settle(w);
      continue;
    }
    double contrib = 0.0;
#pragma unroll
    for (int j = 0; j < kWindow; ++j) {
      const int d = lane + kh::kWave * j;
      if (d < first) {
        contrib += __longlong_as_double((long long)ag[j]);
      } else if (d == first) {
        contrib += __longlong_as_double((long long)inc[j]);
      }
    }
    excl += wave_sum_f64(contrib);
    if (first < kWindow * kh::kWave) return excl;
    end -= kWindow * kh::kWave;
    poll_window(w, s, end, lane);
    settle(w);
  }
}

// A data wave's segment, reduced: per-row lane sums (fp64) and wave scans.
// Writes this lane's row offsets, off[k] = (rows before k) + (lanes before
// this one in row k), to off[k * kMaxThreads] and returns the segment's
// total (the same in every lane). Exact, as every partial sum here is.
__device__ __forceinline__ double reduce_segment(const float (&v)[kPerThread], double *off) {
  double pre = 0.0;
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    const double sk = (((double)v[4 * k] + (double)v[4 * k + 1]) + (double)v[4 * k + 2]) + (double)v[4 * k + 3];
    const double inc = wave_incl_scan_f64(sk);
    off[k * kMaxThreads] = pre + (inc - sk);
    pre += readlane_f64(inc, kh::kWave - 1);
  }
  return pre;
}

// y of a reduced segment: fl32(prefix + row offset + running sum within the
// float4), with `prefix` everything before the segment.
__device__ __forceinline__ void finish_segment(const float (&v)[kPerThread], const double *off, double prefix,
                                               float (&o)[kPerThread]) {
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    double run = prefix + off[k * kMaxThreads];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      run += (double)v[4 * k + j];
      o[4 * k + j] = (float)run;
    }
  }
}

// Tile index of a ticket; tickets past the call's tiles map to ntiles (the
// loop's end marker).
__device__ __forceinline__ int64_t tile_of(uint32_t ticket, uint64_t base, int64_t ntiles) {
  const uint32_t i = ticket - first_ticket(base);
  return (int64_t)i < ntiles ? (int64_t)i : ntiles;
}

// The tile loop of one persistent workgroup, a three-stage pipeline. In
// each iteration the workgroup
//   * finishes tile `tc`: look-back, then y for its elements;
//   * reduces tile `tr` and publishes its aggregate BEFORE that look-back;
//   * has the loads of tile `tn` in flight.
// Reducing (and publishing) one iteration ahead of the look-back means every
// predecessor aggregate a look-back needs went out an iteration earlier, so
// a look-back normally completes on its first poll instead of waiting out
// the publication latency of tiles handed out just before it.
// The last wave is the control wave: it takes tickets and does the
// look-back and never touches tile data; the other (data) waves load,
// reduce and store. The two kinds of wave run loops of their own that meet
// at the same two barriers per iteration (A and B, the same count on both
// sides, from the same shared ticket sequence), so the compiler's wait counts
// for one never cover the other's memory operations. The data waves issue
// their tile loads and stores on every path (a tile that is not there has an
// empty range), so a data wave waits for its tile loads only, with its stores
// left in flight; the control wave waits for its ticket and polls only.
// (One loop for both kinds, with the waits the compiler then has to assume,
// ran 107-108 us at n = 2^26 and 13.4 us at 10^6 against 103 and 12.7 us.)
// Each iteration takes one ticket; its value is first needed at barrier B.
// Deadlock-free: the lowest tile in look-back only needs aggregates of lower
// tiles, and each of those is either finished or in the reduce stage of a
// workgroup that publishes it without waiting on anything.
// The control wave takes the workgroup's tickets after its first one or two,
// so it also counts the workgroup done (count_done), in the step after a
// ticket at or past the last tile came back (the first step when the
// workgroup started with one ticket): its one atomic of a step then goes to
// `done` instead of `counter`. The result lands in s_done[0], the
// workgroup's ticket count in s_done[1], before that step's barrier B.
template <bool VEC>
__device__ __forceinline__ void scan_tiles(const float *__restrict__ X, float *__restrict__ Y, const Session &ses,
                                           int64_t n, int64_t tr, int64_t tn, bool single, uint64_t *s_raw,
                                           double *s_wave_total, double *s_prefix, double *s_off,
                                           uint64_t *s_done, int bd, uint32_t tickets0) {
  const int tid = threadIdx.x;
  const int lane = kh::lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kh::kWave);
  const int ndata = bd / kh::kWave - 1;
  const int64_t tile_elems = (int64_t)ndata * kh::kWave * kPerThread;
  const int64_t ntiles = (n + tile_elems - 1) / tile_elems;

  int64_t tc = -1;  // no tile to finish in the first iteration
  // Tickets are taken until one comes back at or past the last tile (the
  // starting pair included); uniform across the workgroup.
  bool taking = !single && tn < ntiles;
  bool counting = !single && !taking;  // count_done due in the next step
  int slot = 0;
  // After barrier B, for every wave: the tile of the ticket taken in this
  // step (when one was), the ticket state, and the tiles of the next step.
  // False once tc was the workgroup's last tile.
  auto advance = [&](bool take) __attribute__((always_inline)) -> bool {
    const int64_t after =
        take ? tile_of((uint32_t)__builtin_amdgcn_readfirstlane((int)s_raw[slot]), ses.base, ntiles) : ntiles;
    if (take && after >= ntiles) {
      taking = false;  // the workgroup's last ticket is back
      counting = true;
    }
    if (tr >= ntiles) return false;
    tc = tr;
    tr = tn;
    tn = after;
    // s_raw[slot] was read above, after barrier B, and is next written two
    // iterations later. s_wave_total and s_prefix are rewritten only after
    // every wave has passed the next barrier A, past all their reads. A
    // thread's row offsets are its own: buffer `slot` holds tile tr's (read
    // as tile tc's in the next iteration, where slot has flipped).
    slot ^= 1;
    return true;
  };

  if (wave == ndata) {
    // ---- control wave -------------------------------------------------------
    uint32_t tickets = tickets0;  // lane 0: taken so far
    double agg_c = 0.0;    // aggregate of tile tc
    // The ticket counter as a 64-bit word (its low half is the counter), so
    // that a ticket and the done count are one atomic instruction of one
    // width, whose result needs no merge of two values (which would wait
    // for it where it is issued).
    uint64_t *const counter64 = reinterpret_cast<uint64_t *>(&ses.c->counter);
    for (;;) {
      const bool take = taking, count = counting;
      counting = false;
      const bool looks_back = tc > 0;
      // The one atomic of the step: the next ticket, or the done count.
      // Defined only on lane 0, where it is used.
      uint64_t raw;
      if (lane == 0 && (take || count)) {
        raw = fetch_add(take ? counter64 : &ses.c->done, take ? uint64_t(1) : ((uint64_t)tickets << 32) | 1u);
        tickets += take;
      }
      // The first look-back poll for tile tc goes out now, before barrier
      // A: tc was reduced (and its predecessors' aggregates published) in
      // earlier iterations, so its round trip overlaps the data waves'
      // reduction. Always issued; waited for before any branch below.
      Window w;
      poll_window(w, ses, looks_back ? tc - 1 : 0, lane);
      kh::lds_barrier();  // barrier A
      // ---- publish tile tr's aggregate (tile 0: it is its inclusive) -------
      double agg_r = 0.0;
      if (tr < ntiles) agg_r = wave_sum_f64(lane < ndata ? s_wave_total[lane] : 0.0);
      publish(ses.rec, !single && tr < ntiles - 1, tr, tr == 0 ? ses.keys.inc : ses.keys.agg, tag_of(ses.base, tr),
              agg_r, lane);
      // ---- decoupled look-back for tile tc -----------------------------------
      settle(w);
      double excl = 0.0;
      if (looks_back) excl = look_back(ses, tc, lane, w);
      // The atomic went out before the polls just waited for.
      if (lane == 0) {
        *s_prefix = excl;
        s_raw[slot] = take ? raw : 0ull;
        if (count) {
          s_done[0] = raw;
          s_done[1] = tickets;
        }
      }
      publish(ses.rec, looks_back && tc < ntiles - 1, tc, ses.keys.inc, tag_of(ses.base, tc), excl + agg_c, lane);
      agg_c = agg_r;
      kh::lds_barrier();  // barrier B
      if (!advance(take)) return;
    }
  }

  // ---- data waves -------------------------------------------------------------
  const int seg = wave * kh::kWave * kPerThread;  // offset in the tile
  // Per-thread row offsets of a reduced tile wait in LDS for its output
  // stage (two buffers: reduce stage and output stage, alternating).
  double *my_off = s_off + tid;
  // Buffer resource over tile t's elements; empty for a tile that is not there.
  auto span = [&](const float *base, int64_t t) {
    const bool in = t >= 0 && t < ntiles;
    const int64_t at = in ? t * tile_elems : 0;
    return tile_rsrc(base + at, in ? (n - at < tile_elems ? n - at : tile_elems) : 0);
  };
  double wexcl_c = 0.0;  // sum of earlier waves' totals in tile tc

  // One pipeline iteration: finish tc (data in vc), reduce tr (vr), load tn
  // (into vn). False once tc was the workgroup's last tile. The caller
  // rotates the three register buffers instead of copying them.
  auto step = [&](float (&vc)[kPerThread], float (&vr)[kPerThread], float (&vn)[kPerThread])
      __attribute__((always_inline)) -> bool {
    const bool take = taking;
    counting = false;
    if (tr < ntiles) {
      // ---- reduce tile tr -------------------------------------------------
      const double total = reduce_segment(vr, my_off + slot * kRows * kMaxThreads);
      if (lane == 0) s_wave_total[wave] = total;
    }
    kh::lds_barrier();  // barrier A
    // ---- tile tn's loads go out now and land during the look-back ----------
    load_seg<VEC>(vn, span(X, tn), seg, lane);
    double wexcl_r = 0.0;
    if (tr < ntiles)
      for (int w = 0; w < wave; ++w) wexcl_r += s_wave_total[w];
    kh::lds_barrier();  // barrier B
    // ---- y = fl32(prefix + row offset + running sum within the float4) -----
    {
      float o[kPerThread];
      finish_segment(vc, my_off + (slot ^ 1) * kRows * kMaxThreads, *s_prefix + wexcl_c, o);
      store_seg<VEC>(o, span(Y, tc), seg, lane);
    }
    wexcl_c = wexcl_r;
    return advance(take);
  };

  float a[kPerThread], b[kPerThread], c[kPerThread];
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) a[i] = c[i] = 0.0f;
  load_seg<VEC>(b, span(X, tr), seg, lane);
  for (;;) {
    if (!step(a, b, c)) return;
    if (!step(b, c, a)) return;
    if (!step(c, a, b)) return;
  }
}

// A call with a workgroup for every tile (one round): this workgroup's tile
// is `tile`, its data (`v`) already in flight. Wave 0 is the control wave
// here (the first wave of the workgroup to issue, so its header load is not
// queued behind the tile loads of the workgroup's other waves); waves 1 ..
// ndata hold the data, wave w segment w - 1. The data waves reduce the tile
// while the control wave opens the session; after barrier A the control
// wave publishes the aggregate and looks back at once, after barrier B the
// data waves write y while the control wave counts the workgroup done (its
// atomic, on one line every workgroup updates, is off the stores' path).
// (Through the pipelined tile loop such a call took a barrier pair more,
// whose control-wave side waited for a look-back poll of no tile, and the
// session barrier before the reduction: 8.5 us at n = 10^6.)
template <bool VEC>
__device__ __forceinline__ void scan_one_tile(float *__restrict__ Y, Session ses, int64_t n, int64_t tile,
                                              int64_t ntiles, uint32_t nblocks, int bd, float (&v)[kPerThread],
                                              double *s_wave_total, double *s_prefix, double *s_off) {
  const int tid = threadIdx.x;
  const int lane = kh::lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kh::kWave);
  const int ndata = bd / kh::kWave - 1;
  const int64_t tile_elems = (int64_t)ndata * kh::kWave * kPerThread;
  if (wave == 0) {
    // ---- control wave -------------------------------------------------------
    const Opened o = open_session(ses.h, ses.c, ntiles, nblocks, 0, lane);
    const bool ok = __builtin_amdgcn_readfirstlane((int)o.ok) != 0;
    const uint64_t nonce = readlane_u64(o.nonce, 0);
    ses.base = readlane_u64(o.base, 0);
    ses.keys = record_keys(session_key(ses.h, nonce));
    kh::lds_barrier();  // barrier A: the data waves' totals are in LDS
    double excl = __builtin_nan("");
    if (ok) {
      const double agg = wave_sum_f64(lane < ndata ? s_wave_total[lane] : 0.0);
      publish(ses.rec, tile < ntiles - 1, tile, tile == 0 ? ses.keys.inc : ses.keys.agg, tag_of(ses.base, tile),
              agg, lane);
      excl = 0.0;
      if (tile > 0) {
        // Every tile of the call publishes its aggregate at about this
        // moment; a poll issued at once mostly finds its predecessors' not
        // yet visible and polls again, a round trip later. Waiting ~0.4 us
        // first (16 x 64 clocks) measured 7.34 against 7.54 us at n = 10^6.
        __builtin_amdgcn_s_sleep(16);
        Window w;
        poll_window(w, ses, tile - 1, lane);
        settle(w);
        excl = look_back(ses, tile, lane, w);
        publish(ses.rec, tile < ntiles - 1, tile, ses.keys.inc, tag_of(ses.base, tile), excl + agg, lane);
      }
    }
    if (lane == 0) *s_prefix = excl;
    kh::lds_barrier();  // barrier B
    if (ok && lane == 0) close_session(ses.h, ses.c, ses.base, nonce, count_done(ses.c, 0), 0, nblocks);
    return;
  }
  // ---- data waves -------------------------------------------------------------
  const int d = wave - 1;  // segment index
  double *my_off = s_off + tid;
  const double total = reduce_segment(v, my_off);
  if (lane == 0) s_wave_total[d] = total;
  kh::lds_barrier();  // barrier A
  double wexcl = 0.0;
  for (int w = 0; w < d; ++w) wexcl += s_wave_total[w];
  kh::lds_barrier();  // barrier B
  float o[kPerThread];
  finish_segment(v, my_off, *s_prefix + wexcl, o);
  const int64_t at = tile * tile_elems;
  store_seg<VEC>(o, tile_rsrc(Y + at, n - at < tile_elems ? n - at : tile_elems), d * kh::kWave * kPerThread, lane);
}

// First 8-byte boundary of a float buffer (0 or 1 floats in), by pointer
// arithmetic so that the compiler keeps the global address space.
template <typename T>
__device__ __forceinline__ T *align8(float *p) {
  return reinterpret_cast<T *>(p + ((reinterpret_cast<uintptr_t>(p) >> 2) & 1));
}

// Bytes of a unit-stride float buffer from its first 8-byte boundary.
__device__ __forceinline__ int64_t bytes_from_align8(const float *p, int64_t n0, int64_t s0) {
  if (n0 > 1 && s0 != 1) return 0;
  return 4 * (n0 - (int64_t)((reinterpret_cast<uintptr_t>(p) >> 2) & 1));
}

}  // namespace

extern "C" __global__ void __launch_bounds__(kMaxThreads)
scan(KH_MEMREF1(const float, x), KH_MEMREF1(float, y), KH_MEMREF1(float, y_lo),
     KH_MEMREF1(float, totals_hi), KH_MEMREF1(float, totals_lo)) {
  (void)y_lo_alloc;
  (void)y_lo_base;
  const float *__restrict__ X = KH_PTR(x);
  float *__restrict__ Y = KH_PTR(y);
  const int64_t n = x_n0;
  const int tid = threadIdx.x;

  __shared__ int64_t s_ticket[2];
  __shared__ uint64_t s_raw[2];
  __shared__ uint64_t s_session[3];  // base, session key, nonce
  __shared__ double s_wave_total[kMaxThreads / kh::kWave];
  __shared__ double s_off[2 * kRows * kMaxThreads];
  __shared__ double s_prefix;

  if (n <= 0) return;
  // Every argument and the launch geometry in one round of scalar loads.
  const uint32_t gxy = kh::group_size_word(), gzw = kh::group_size_z_word();
  const uint32_t bx = kh::grid_blocks_x(), by = kh::grid_blocks_y(), bz = kh::grid_blocks_z();
  KH_ARGS_READY(x_base, x_off, y_base, y_off, totals_hi_base, totals_hi_off, totals_hi_n0, totals_hi_s0,
                totals_lo_base, totals_lo_off, totals_lo_n0, totals_lo_s0, gxy, gzw, bx, by, bz);
  const uint32_t nblocks = bx * by * bz;
  // Refusals, decided identically by every workgroup before any state is
  // touched: the launch shape the tile loop assumes (one-dimensional
  // workgroups of whole waves, at least three data waves) and room for the
  // header and the records. y := NaN, never a hang or a stray write.
  const int bdx = (int)kh::threads_x_of(gxy);
  const bool shape_ok = (bdx >= kMinThreads) & (bdx % kh::kWave == 0) & (kh::threads_y_of(gxy) == 1) &
                        (kh::threads_z_of(gzw) == 1);
  const int64_t tile_elems = (int64_t)(bdx - kh::kWave) * kPerThread;
  const int64_t ntiles = shape_ok ? (n + tile_elems - 1) / tile_elems : 0;
  const int64_t lo_bytes = bytes_from_align8(KH_PTR(totals_lo), totals_lo_n0, totals_lo_s0);
  // (Tickets and tile indices are 32-bit and records are addressed with
  // 32-bit byte offsets below 2^31: ntiles < 2^27, which always holds for a
  // device's memory (2^27 tiles of at least 3072 elements); refused
  // otherwise.)
  const bool room = ntiles < (int64_t(1) << 27) && (ntiles == 1 ||
                    (lo_bytes >= (int64_t)(sizeof(Header) + sizeof(Counters)) &&
                     bytes_from_align8(KH_PTR(totals_hi), totals_hi_n0, totals_hi_s0) >=
                         (int64_t)sizeof(Record) * (ntiles - 1)));
  __shared__ bool s_refuse;
  bool refuse = !shape_ok || !room;
  Session ses{align8<Header>(KH_PTR(totals_lo)), nullptr, align8<Record>(KH_PTR(totals_hi)), 0, Keys{0, 0}};
  ses.c = counters_of(ses.h, lo_bytes);
  const bool single = ntiles == 1;  // one tile: one workgroup, no look-back state
  const bool vec = kh::aligned16(X) && kh::aligned16(Y) && (n & 3) == 0;
  const int ctl = bdx - kh::kWave;  // first thread of the control wave
  const int64_t block = ((int64_t)blockIdx.z * by + blockIdx.y) * bx + blockIdx.x;
  // How tiles are handed out:
  //   * when the grid has a workgroup for every tile (one round), tile i
  //     goes to the workgroup of flat index i: no ticket, and the data
  //     waves issue the tile's loads at once, while the control wave reads
  //     the session. A tile waits only on tiles of lower index, so the
  //     lowest unfinished tile waits on nothing: its workgroup is running,
  //     or waits to start on its XCD behind workgroups of lower index only
  //     (each XCD starts its workgroups in index order), which finish
  //     first. Every wait ends (and is bounded besides);
  //   * otherwise by atomic tickets, two to start with (the second tile's
  //     loads then go out in the first step).
  const bool by_index = !single && ntiles <= (int64_t)nblocks;
  const uint32_t tickets0 = by_index ? 0 : 2;
  float first_data[kPerThread];
  if (!refuse && by_index && block < ntiles && tid >= kh::kWave) {
    // (Wave 0 is the control wave of a one-tile call; wave w loads segment w - 1.)
    const int64_t at = block * tile_elems;
    const __amdgpu_buffer_rsrc_t r = tile_rsrc(X + at, n - at < tile_elems ? n - at : tile_elems);
    const int seg = (tid / kh::kWave - 1) * kh::kWave * kPerThread;
    if (vec)
      load_seg<true>(first_data, r, seg, kh::lane_id());
    else
      load_seg<false>(first_data, r, seg, kh::lane_id());
  }
  if (!refuse && by_index) {
    if (block >= ntiles) {
      // No tile for this workgroup: count it done (the call closes when
      // every workgroup has).
      if (tid < kh::kWave) {
        const Opened o = open_session(ses.h, ses.c, ntiles, nblocks, 0, kh::lane_id());
        if (kh::lane_id() == 0 && o.ok) close_session(ses.h, ses.c, o.base, o.nonce, count_done(ses.c, 0), 0, nblocks);
      }
      return;
    }
    if (vec)
      scan_one_tile<true>(Y, ses, n, block, ntiles, nblocks, bdx, first_data, s_wave_total, &s_prefix, s_off);
    else
      scan_one_tile<false>(Y, ses, n, block, ntiles, nblocks, bdx, first_data, s_wave_total, &s_prefix, s_off);
    return;
  }
  if (!refuse && !single) {
    // Wave 0 opens the session (it waits at the barrier below like every
    // data wave; the control wave then starts its loop with no round trip
    // behind it: 99.5 against 100.5 us at n = 2^26).
    if (tid < kh::kWave) {
      const Opened o = open_session(ses.h, ses.c, ntiles, nblocks, tickets0, kh::lane_id());
      if (tid == 0) {
        s_session[0] = o.base;
        s_session[1] = session_key(ses.h, o.nonce);
        s_session[2] = o.nonce;
        s_ticket[0] = tile_of(o.t0, o.base, ntiles);
        s_ticket[1] = tile_of(o.t1, o.base, ntiles);
        s_refuse = !o.ok;
      }
    }
    kh::lds_barrier();
    refuse = s_refuse;
  }
  if (refuse) {
    const int64_t ty = kh::threads_y_of(gxy), tz = kh::threads_z_of(gzw);
    const int64_t threads = (int64_t)bdx * ty * tz;
    const int64_t flat = ((int64_t)threadIdx.z * ty + threadIdx.y) * bdx + tid;
    const int64_t blocks = nblocks;
    for (int64_t i = block * threads + flat; i < n; i += blocks * threads) Y[i] = __builtin_nanf("");
    return;
  }
  if (single) {
    if (block != 0) return;
    s_ticket[0] = 0;
    s_ticket[1] = ntiles;
    s_session[0] = 0;
    s_session[1] = 0;
    kh::lds_barrier();
  }
  const int64_t first = s_ticket[0];
  const int64_t second = s_ticket[1];
  ses.base = s_session[0];
  ses.keys = record_keys(s_session[1]);
  if (first >= ntiles) {
    // No tile for this workgroup: both its tickets are past the end.
    if (tid == ctl) close_session(ses.h, ses.c, ses.base, s_session[2], count_done(ses.c, tickets0), tickets0, nblocks);
    return;
  }
  __shared__ uint64_t s_done[2];
  if (vec)
    scan_tiles<true>(X, Y, ses, n, first, second, single, s_raw, s_wave_total, &s_prefix, s_off, s_done, bdx,
                     tickets0);
  else
    scan_tiles<false>(X, Y, ses, n, first, second, single, s_raw, s_wave_total, &s_prefix, s_off, s_done, bdx,
                      tickets0);
  // s_done and s_session were written before the last barrier B.
  if (!single && tid == ctl)
    close_session(ses.h, ses.c, ses.base, s_session[2], s_done[0], (uint32_t)s_done[1], nblocks);
}

// The reference's second pass (scan.cpp:350-453). With the single-pass
// `scan`, y is already final: this kernel leaves y and the totals unchanged
// and writes each 256-element block's exclusive offset (off_hi = y[256 b - 1],
// the fp32 rounding of the exact exclusive prefix; off_lo = off_lo2 = 0).
extern "C" __global__ void __launch_bounds__(256)
scan_totals(KH_MEMREF1(float, totals_hi), KH_MEMREF1(float, totals_lo), KH_MEMREF1(float, off_hi),
            KH_MEMREF1(float, off_lo), KH_MEMREF1(float, off_lo2), KH_MEMREF1(float, y),
            KH_MEMREF1(float, y_lo)) {
  (void)totals_hi_alloc;
  (void)totals_lo_alloc;
  const int64_t n = y_n0;
  const int64_t T = off_hi_n0;
  const float *__restrict__ Y = KH_PTR(y);
  float *__restrict__ oh = KH_PTR(off_hi);
  float *__restrict__ ol = KH_PTR(off_lo);
  float *__restrict__ ol2 = KH_PTR(off_lo2);
  const int64_t stride = (int64_t)blockDim.x * gridDim.x;
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < T; b += stride) {
    oh[b] = (b == 0 || b * 256 > n) ? 0.0f : Y[b * 256 - 1];
    ol[b] = 0.0f;
    ol2[b] = 0.0f;
  }
}
