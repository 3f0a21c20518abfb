// Allowed-token masks of the schema-constrained tool-call grammar on the
// device: one thread per token piece runs the grammar from the current
// state over the piece's bytes (tools/agent.ts:164-175 asks this of a
// grammar clone for every piece; tools/grammar.ts defines the automaton).
//
// The host compiles the tool schemas once into a program (schema nodes,
// value-frame descriptors, property names, enum/const candidates, tool
// names) and serializes the grammar state each step (tool-call phase and
// the JSON frame stack).  Layouts are the ones documented in
// include/needle_hip.h.  The interpreter follows grammar.ts byte for byte,
// including its retry limits; three outcomes per piece: accepted, rejected,
// or undecided when the answer needs a check this kernel does not make.  It
// decides a closing string's minLength / maxLength (code points as
// Array.from counts them), pattern (an automaton the host builds from the
// JavaScript regular expression, stepped per UTF-16 code unit) and email /
// uuid formats, and a completed number's finiteness, integrality, bounds and
// multipleOf whenever its value is exact in the fast path (at most 2^53
// significant, a decimal exponent within +-22); it leaves undecided a string
// under enum / const or under a pattern with no automaton, a number under
// enum / const or outside the fast path, a composite value closing under
// enum / const, an array under uniqueItems closing in the piece that
// completed an item (the host tells whether the items it holds are
// distinct), and a stack deeper than kMaxDepth.  The host
// grammar settles the undecided pieces.
#include <cstring>
#include <vector>

#include "nd_internal.hpp"

namespace {

constexpr int kGThreads = 256;
constexpr uint32_t kMaxDepth = 24;

enum Kind : uint32_t { kValue = 1, kString, kNumber, kLiteral, kChoice, kArray, kObject, kKey };
enum VKind : uint32_t { vString = 0, vNumber, vBoolean, vNull, vArray, vObject };
enum TypeBit : uint32_t { tString = 1, tNumber = 2, tInteger = 4, tBoolean = 8, tNull = 16,
                          tArray = 32, tObject = 64 };
enum NodeFlag : uint32_t { fStrCheck = 1, fNumCheck = 2, fIntOnly = 4, fValueCheck = 8,
                           fUnique = 16 };
// An array frame's word 2: bit 0 = its items are the host state's (none
// completed since), bit 1 = those items are pairwise distinct by their JSON
// text (grammar.ts uniqueItems), as the host computed them.
constexpr uint32_t kItemsHost = 1, kItemsUnique = 2;
// A node's entry: words 0..11 its structure, words 12..27 its value checks
// (flags below, minLength, maxLength, 0, then minimum, maximum,
// exclusiveMinimum, exclusiveMaximum, multipleOf as float64, low word first).
constexpr uint32_t kNodeWords = 28;
enum Check : uint32_t {
  kcMinLength = 1, kcMaxLength = 2, kcEmail = 4, kcUuid = 8, kcStringHost = 16, kcPattern = 32,
  kcMinimum = 256, kcMaximum = 512, kcExclusiveMinimum = 1024, kcExclusiveMaximum = 2048,
  kcMultipleOf = 4096, kcNumberHost = 8192
};
constexpr uint32_t kLengthMax = 0xFFFFFF;               // string lengths are counted up to this
constexpr uint64_t kMantissaCap = 1000000000000000000ull;  // digits taken while below this
enum Tool : uint32_t { pArrayOpen = 0, pCallOpen, pNameLiteral, pToolName, pArgsLiteral, pArgs,
                       pCallClose, pAfterCall, pDone };
enum Res : int { rReject = 0, rOk = 1, rUndecided = 2 };

struct Program {
  const uint32_t* nodes;   // [n][12]
  const uint32_t* values;  // [n][4]
  const uint32_t* alts;    // node indices
  const uint32_t* props;   // [n][4]
  const uint32_t* cands;   // [n][4]
  const uint32_t* tools;   // [n][4]
  const uint8_t* bytes;
  const uint32_t* regex;  // pattern automata
  uint32_t n_nodes, n_values, n_tools;  // bounds for indices that come from the state
};

// Node fields.
__device__ __forceinline__ uint32_t nd_types(const Program& p, uint32_t n) {
  return p.nodes[n * kNodeWords];
}
__device__ __forceinline__ uint32_t nd_flags(const Program& p, uint32_t n) {
  return p.nodes[n * kNodeWords + 1];
}

// The pattern automaton of node n (node word 15 holds its offset in the
// automata + 1, or 0).  An automaton: [states, classes, bounds, 0], then the
// bounds (first code unit | class << 16, ascending from unit 0), a flag per
// state (bit 0: the value read so far matches the pattern), and the next
// state per (state, class).  State 0 is the start of a value.
__device__ __forceinline__ const uint32_t* nd_regex(const Program& p, uint32_t n) {
  const uint32_t o = p.nodes[n * kNodeWords + 15];
  return o ? p.regex + (o - 1) : nullptr;
}

__device__ uint32_t regex_step(const uint32_t* rx, uint32_t state, uint32_t unit) {
  const uint32_t nb = rx[2];
  const uint32_t* b = rx + 4;
  uint32_t lo = 0, hi = nb;  // the last bound whose first unit is <= unit
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if ((b[mid] & 0xFFFFu) <= unit)
      lo = mid;
    else
      hi = mid;
  }
  return rx[4 + nb + rx[0] + state * rx[1] + (b[lo] >> 16)];
}

// acc: the running summary of the string or number in progress (always the
// top frame), zeroed when one starts.  String: code points so far (an
// escaped high surrogate followed by an escaped low one counts once, as
// Array.from counts the decoded value), word 1 = the \u value being read
// (bits 0-15) | an escaped high surrogate pending (16) | email state
// (17-19) | uuid position (20-25) | uuid mismatch (26), the UTF-8 code point
// being assembled, the pattern automaton's state.  Number: mantissa m (words 0, 1) of the significant
// digits taken while m < 10^18, k (word 2, two's complement) with value =
// m 10^(k + exponent), word 3 = exponent digits (saturating at 999999) |
// minus (24) | exponent minus (25) | a nonzero digit dropped (26).
struct State {
  uint32_t phase, lit, name_live, name_off, cur_tool, used_tools, n_calls, max_calls, n_tools;
  uint32_t args_present, args_complete, args_kind, depth;
  uint32_t acc[4];
  uint32_t fr[kMaxDepth][4];
};

__device__ __forceinline__ uint32_t fkind(const uint32_t* f) { return f[0] & 0xFF; }
__device__ __forceinline__ uint32_t fphase(const uint32_t* f) { return (f[0] >> 8) & 0xFF; }
__device__ __forceinline__ void set_phase(uint32_t* f, uint32_t ph) {
  f[0] = (f[0] & ~0xFF00u) | (ph << 8);
}

// Bytes that may start a value of each type (grammar.ts:168-177).
__device__ __forceinline__ uint32_t types_for_byte(uint32_t b) {
  if (b == 0x22) return tString;
  if (b == 0x7B) return tObject;
  if (b == 0x5B) return tArray;
  if (b == 0x74 || b == 0x66) return tBoolean;
  if (b == 0x6E) return tNull;
  if (b == 0x2D || (b >= 0x30 && b <= 0x39)) return tNumber | tInteger;
  return 0;
}

// UTF-8 well-formedness of a string's bytes (TextDecoder fatal).  States:
// 0 boundary, 1-3 continuation bytes left, 4 after E0, 5 after ED, 6 after
// F0, 7 after F4, 8 error (sticky).
__device__ __forceinline__ uint32_t utf8_step(uint32_t s, uint32_t b) {
  switch (s) {
    case 0:
      if (b < 0x80) return 0;
      if (b >= 0xC2 && b <= 0xDF) return 1;
      if (b == 0xE0) return 4;
      if (b == 0xED) return 5;
      if (b >= 0xE1 && b <= 0xEF) return 2;
      if (b == 0xF0) return 6;
      if (b >= 0xF1 && b <= 0xF3) return 3;
      if (b == 0xF4) return 7;
      return 8;
    case 1: return b >= 0x80 && b <= 0xBF ? 0 : 8;
    case 2: return b >= 0x80 && b <= 0xBF ? 1 : 8;
    case 3: return b >= 0x80 && b <= 0xBF ? 2 : 8;
    case 4: return b >= 0xA0 && b <= 0xBF ? 1 : 8;
    case 5: return b >= 0x80 && b <= 0x9F ? 1 : 8;
    case 6: return b >= 0x90 && b <= 0xBF ? 2 : 8;
    case 7: return b >= 0x80 && b <= 0x8F ? 2 : 8;
    default: return 8;
  }
}

// JSON number prefix scan as a DFA (isNumberPrefix, grammar.ts:229-254):
// 0 empty, 1 '-', 2 '0', 3 integer digits, 4 '.', 5 fraction digits, 6 'e',
// 7 exponent sign, 8 exponent digits; 10-12 the same exponent states after
// a '.' with no fraction digit ("1.e5" is a prefix the scan accepts but
// never a complete number); 9 = not a prefix.  Complete numbers
// (grammar.ts:256-258) end in 2, 3, 5 or 8.
__device__ __forceinline__ uint32_t number_step(uint32_t s, uint32_t b) {
  const bool digit = b >= 0x30 && b <= 0x39, e = b == 0x65 || b == 0x45;
  const bool sign = b == 0x2B || b == 0x2D, dot = b == 0x2E;
  switch (s) {
    case 0: return b == 0x2D ? 1 : (b == 0x30 ? 2 : (digit ? 3 : 9));
    case 1: return b == 0x30 ? 2 : (digit ? 3 : 9);
    case 2: return dot ? 4 : (e ? 6 : 9);
    case 3: return digit ? 3 : (dot ? 4 : (e ? 6 : 9));
    case 4: return digit ? 5 : (e ? 10 : 9);
    case 5: return digit ? 5 : (e ? 6 : 9);
    case 6: return sign ? 7 : (digit ? 8 : 9);
    case 7: return digit ? 8 : 9;
    case 8: return digit ? 8 : 9;
    case 10: return sign ? 11 : (digit ? 12 : 9);
    case 11: return digit ? 12 : 9;
    case 12: return digit ? 12 : 9;
    default: return 9;
  }
}

// ECMAScript's \s: WhiteSpace (TAB, VT, FF, SP, NBSP, ZWNBSP, the Zs
// category) and LineTerminator (LF, CR, LS, PS).
__device__ __forceinline__ bool js_space(uint32_t c) {
  return (c >= 0x09 && c <= 0x0D) || c == 0x20 || c == 0xA0 || c == 0x1680 ||
         (c >= 0x2000 && c <= 0x200A) || c == 0x2028 || c == 0x2029 || c == 0x202F ||
         c == 0x205F || c == 0x3000 || c == 0xFEFF;
}

// /^[^\s@]+@[^\s@]+\.[^\s@]+$/ (grammar.ts:191) one character at a time: 0
// start, 1 local part, 2 after '@', 3 domain, 4 after a usable '.', 5
// accepting, 6 dead.
__device__ __forceinline__ uint32_t email_step(uint32_t s, uint32_t c) {
  const bool at = c == 0x40, other = !at && !js_space(c);
  switch (s) {
    case 0: return other ? 1 : 6;
    case 1: return other ? 1 : (at ? 2 : 6);
    case 2: return other ? 3 : 6;
    case 3: return other ? (c == 0x2E ? 4 : 3) : 6;
    case 4:
    case 5: return other ? 5 : 6;
    default: return 6;
  }
}

// /^[0-9a-f]{8}-[0-9a-f]{4}-[1-8][0-9a-f]{3}-[89ab][0-9a-f]{3}-[0-9a-f]{12}$/i
// (grammar.ts:192-196): whether character c fits position p.
__device__ __forceinline__ bool uuid_char(uint32_t p, uint32_t c) {
  if (p == 8 || p == 13 || p == 18 || p == 23) return c == 0x2D;
  if (p == 14) return c >= 0x31 && c <= 0x38;
  if (p == 19) return c == 0x38 || c == 0x39 || c == 0x61 || c == 0x62 || c == 0x41 || c == 0x42;
  return (c >= 0x30 && c <= 0x39) || (c >= 0x61 && c <= 0x66) || (c >= 0x41 && c <= 0x46);
}

// One UTF-16 code unit (or one code point above U+FFFF) of the string's
// decoded value into acc; uesc: it came from a \u escape; rx: the string's
// pattern automaton, which reads a code point above U+FFFF as its two
// surrogates (RegExp without the u flag reads code units).
__device__ void string_emit(uint32_t* acc, uint32_t cu, bool uesc, const uint32_t* rx) {
  if (rx) {
    if (cu > 0xFFFFu) {
      acc[3] = regex_step(rx, acc[3], 0xD800u + ((cu - 0x10000u) >> 10));
      acc[3] = regex_step(rx, acc[3], 0xDC00u + ((cu - 0x10000u) & 0x3FFu));
    } else {
      acc[3] = regex_step(rx, acc[3], cu);
    }
  }
  uint32_t w = acc[1];
  if (((w >> 16) & 1) && uesc && cu >= 0xDC00 && cu <= 0xDFFF) {
    w &= ~(1u << 16);  // the low half of an escaped pair: one code point
  } else {
    if (acc[0] < kLengthMax) acc[0] += 1;
    w = (w & ~(1u << 16)) | ((uesc && cu >= 0xD800 && cu <= 0xDBFF) ? 1u << 16 : 0u);
  }
  const uint32_t email = email_step((w >> 17) & 7, cu);
  uint32_t pos = (w >> 20) & 63, miss = (w >> 26) & 1;
  if (!miss) {
    if (pos < 36 && uuid_char(pos, cu))
      pos += 1;
    else
      miss = 1;
  }
  acc[1] = (w & 0x1FFFFu) | (email << 17) | (pos << 20) | (miss << 26);
}

// The checks of a string closing under node n (validateString,
// grammar.ts:179-203) that the kernel makes; enum / const, and a pattern
// without an automaton, are the host's.
__device__ int string_checks(const Program& P, uint32_t n, const uint32_t* acc,
                             const uint32_t* rx) {
  const uint32_t* c = P.nodes + n * kNodeWords + 12;
  const uint32_t cf = c[0], len = acc[0];
  if (cf & kcStringHost) return rUndecided;
  if ((cf & kcPattern) && !(rx[4 + rx[2] + acc[3]] & 1u)) return rReject;
  if ((cf & (kcMinLength | kcMaxLength)) && len >= kLengthMax) return rUndecided;
  if ((cf & kcMinLength) && len < c[1]) return rReject;
  if ((cf & kcMaxLength) && len > c[2]) return rReject;
  if ((cf & kcEmail) && ((acc[1] >> 17) & 7) != 5) return rReject;
  if ((cf & kcUuid) && (((acc[1] >> 20) & 63) != 36 || ((acc[1] >> 26) & 1))) return rReject;
  return rOk;
}

__constant__ const double kPow10[23] = {1e0,  1e1,  1e2,  1e3,  1e4,  1e5,  1e6,  1e7,
                                        1e8,  1e9,  1e10, 1e11, 1e12, 1e13, 1e14, 1e15,
                                        1e16, 1e17, 1e18, 1e19, 1e20, 1e21, 1e22};

// Number(text) from the accumulator when it is exact in the fast path: a
// mantissa of at most 2^53 times an exactly representable power of ten
// (10^0 .. 10^22), one correctly rounded product or quotient -- the value
// a correctly rounding Number() gives.  False: outside the fast path.
__device__ bool number_value(const uint32_t* acc, double* v) {
  const uint64_t m = (uint64_t)acc[0] | ((uint64_t)acc[1] << 32);
  const uint32_t w = acc[3];
  if (w & (1u << 26)) return false;
  double r = 0.0;
  if (m != 0) {
    const int32_t e = (int32_t)(w & 0xFFFFFFu);
    const int64_t K = (int64_t)(int32_t)acc[2] + (((w >> 25) & 1) ? -e : e);
    if (m > (1ull << 53) || K < -22 || K > 22) return false;
    r = K >= 0 ? (double)m * kPow10[K] : (double)m / kPow10[-K];
  }
  *v = ((w >> 24) & 1) ? -r : r;
  return true;
}

__device__ __forceinline__ double word_double(const uint32_t* p) {
  return __builtin_bit_cast(double, (uint64_t)p[0] | ((uint64_t)p[1] << 32));
}

// validateNumber (grammar.ts:205-222) of a finite value under node n.
__device__ int number_checks(const Program& P, uint32_t n, uint32_t nf, double v) {
  if ((nf & fIntOnly) && v != floor(v)) return rReject;  // Number.isInteger
  if (!(nf & fNumCheck)) return rOk;
  const uint32_t* c = P.nodes + n * kNodeWords + 12;
  const uint32_t cf = c[0];
  if (cf & kcNumberHost) return rUndecided;
  if ((cf & kcMinimum) && v < word_double(c + 4)) return rReject;
  if ((cf & kcMaximum) && v > word_double(c + 6)) return rReject;
  if ((cf & kcExclusiveMinimum) && v <= word_double(c + 8)) return rReject;
  if ((cf & kcExclusiveMaximum) && v >= word_double(c + 10)) return rReject;
  if (cf & kcMultipleOf) {
    const double q = v / word_double(c + 12);
    double r = q;  // Math.round: nearest integer, ties toward +Infinity
    if (isfinite(q)) {
      r = floor(q);
      if (q - r >= 0.5) r += 1.0;
    }
    const double aq = fabs(q);
    const double scale = aq != aq ? aq : (aq > 1.0 ? aq : 1.0);  // Math.max(1, |q|)
    if (fabs(q - r) > 1e-9 * scale) return rReject;
  }
  return rOk;
}

// #finish (grammar.ts:633-656): pop the frame; the parent takes the value
// (the whole arguments value when the stack empties).
__device__ int finish(State& st, uint32_t vkind) {
  st.depth -= 1;
  if (st.depth == 0) {
    st.args_complete = 1;
    st.args_kind = vkind;
    return rOk;
  }
  uint32_t* parent = st.fr[st.depth - 1];
  if (fkind(parent) == kArray && fphase(parent) == 2) {
    parent[3] += 1;
    parent[2] &= ~kItemsHost;  // an item the host has not compared
    set_phase(parent, 3);
    return rOk;
  }
  if (fkind(parent) == kObject && fphase(parent) == 5 && parent[3] < 32) {
    parent[2] |= 1u << parent[3];
    parent[3] = 0xFFFFFFFFu;
    set_phase(parent, 6);
    return rOk;
  }
  return rReject;  // inconsistent stack: the reference throws
}

// JsonSchemaGrammar.feedByte (grammar.ts:297-631).
__device__ int json_byte(const Program& P, State& st, uint32_t b) {
  if (st.args_complete) return rReject;
  for (int retry = 0; retry < 16; ++retry) {
    if (st.depth == 0) return rReject;
    uint32_t* f = st.fr[st.depth - 1];
    // Indices read from the serialized state stay inside the program.
    const uint32_t kind = fkind(f);
    if (kind == kValue || kind == kChoice ? f[1] >= P.n_values
                                          : (kind != kLiteral && f[1] >= P.n_nodes))
      return rReject;
    switch (kind) {
      case kValue: {
        const uint32_t* v = P.values + f[1] * 4;
        if (v[0] == 1) {  // every alternative is const/enum: a choice over their JSON
          f[0] = kChoice;
          f[2] = v[2] >= 32 ? 0xFFFFFFFFu : ((1u << v[2]) - 1u);
          f[3] = 0;
          continue;
        }
        if (v[0] == 2) return rUndecided;  // more candidates than the mask holds
        const uint32_t want = types_for_byte(b);
        uint32_t node = 0xFFFFFFFFu;
        for (uint32_t i = 0; i < v[2]; ++i) {
          const uint32_t n = P.alts[v[1] + i];
          if (nd_types(P, n) & want) {
            node = n;
            break;
          }
        }
        if (node == 0xFFFFFFFFu) return rReject;
        if (b == 0x22) {
          f[0] = kString;
          f[1] = node;
          f[2] = 0;
          f[3] = 0;
          st.acc[0] = st.acc[1] = st.acc[2] = st.acc[3] = 0;
        } else if (want & tNumber) {
          f[0] = kNumber;  // DFA state 0 in the phase byte
          f[1] = node;
          f[2] = 0;
          f[3] = 0;
          st.acc[0] = st.acc[1] = st.acc[2] = st.acc[3] = 0;
        } else if (want == tBoolean) {
          f[0] = kLiteral;
          f[1] = b == 0x74 ? 0 : 1;
          f[3] = 0;
        } else if (want == tNull) {
          f[0] = kLiteral;
          f[1] = 2;
          f[3] = 0;
        } else if (want == tArray) {
          f[0] = kArray;
          f[1] = node;
          f[3] = 0;
        } else {
          f[0] = kObject;
          f[1] = node;
          f[2] = 0;
          f[3] = 0xFFFFFFFFu;
        }
        continue;
      }
      case kString: {
        // Flags: bit 0 started, bit 1 escaped, bits 2-4 \u hex digits left,
        // bits 8-11 the UTF-8 state of every byte taken so far.
        const uint32_t flags = f[0] >> 16;
        const bool started = flags & 1, escaped = flags & 2;
        uint32_t uni = (flags >> 2) & 7;
        if (!started) {
          if (b != 0x22) return rReject;
          f[0] = kString | (1u << 16);
          return rOk;
        }
        const uint32_t* rx = nd_regex(P, f[1]);
        if (rx && st.acc[3] >= rx[0]) return rReject;  // not a state of the automaton
        const uint32_t prev8 = (flags >> 8) & 15, u8 = utf8_step(prev8, b);
        if (uni > 0) {
          const bool digit = b >= 0x30 && b <= 0x39, upper = b >= 0x41 && b <= 0x46,
                     lower = b >= 0x61 && b <= 0x66;
          if (!(digit || upper || lower)) return rReject;
          uni -= 1;
          const uint32_t hv =
              ((st.acc[1] << 4) | (digit ? b - 0x30 : (b | 0x20u) - 0x57)) & 0xFFFFu;
          st.acc[1] = (st.acc[1] & ~0xFFFFu) | hv;
          if (uni == 0) string_emit(st.acc, hv, true, rx);
          f[0] = kString | ((1u | (uni << 2) | (u8 << 8)) << 16);
          return rOk;
        }
        if (escaped) {
          if (!(b == 0x22 || b == 0x5C || b == 0x2F || b == 0x62 || b == 0x66 || b == 0x6E ||
                b == 0x72 || b == 0x74 || b == 0x75))
            return rReject;
          uni = b == 0x75 ? 4 : 0;
          if (uni)
            st.acc[1] &= ~0xFFFFu;
          else  // the escape's character
            string_emit(st.acc,
                        b == 0x62   ? 0x08u
                        : b == 0x66 ? 0x0Cu
                        : b == 0x6E ? 0x0Au
                        : b == 0x72 ? 0x0Du
                        : b == 0x74 ? 0x09u
                                    : b,
                        false, rx);
          f[0] = kString | ((1u | (uni << 2) | (u8 << 8)) << 16);
          return rOk;
        }
        if (b == 0x5C) {
          f[0] = kString | ((1u | 2u | (u8 << 8)) << 16);
          return rOk;
        }
        if (b < 0x20) return rReject;
        if (b != 0x22) {
          if (prev8 == 0) {
            if (b < 0x80)
              string_emit(st.acc, b, false, rx);
            else
              st.acc[2] = b & (b < 0xE0 ? 0x1Fu : (b < 0xF0 ? 0x0Fu : 0x07u));
          } else {
            st.acc[2] = ((st.acc[2] << 6) | (b & 0x3Fu)) & 0x1FFFFFu;
            if (u8 == 0) string_emit(st.acc, st.acc[2], false, rx);
          }
          f[0] = kString | ((1u | (u8 << 8)) << 16);
          return rOk;
        }
        // Closing quote: the bytes must decode (fatal UTF-8), then the
        // string's schema checks.
        if (u8 != 0) return rReject;
        if (nd_flags(P, f[1]) & fStrCheck) {
          const int r = string_checks(P, f[1], st.acc, rx);
          if (r != rOk) return r;
        }
        return finish(st, vString) == rOk ? rOk : rReject;
      }
      case kNumber: {
        const uint32_t s = fphase(f);
        const bool numeric = (b >= 0x30 && b <= 0x39) || b == 0x65 || b == 0x45 || b == 0x2B ||
                             b == 0x2D || b == 0x2E;
        if (numeric) {
          const uint32_t n = number_step(s, b);
          if (n == 9) return rReject;
          uint32_t flags = f[0] >> 16;
          if (n == 6 || n == 10) flags |= 1;           // exponent seen
          if (n == 5 && b != 0x30) flags |= 2;         // nonzero fraction digit
          if ((n == 2 || n == 3) && f[3] < 1000) f[3] += 1;  // integer digits
          f[0] = kNumber | (n << 8) | (flags << 16);
          // The value: integer and fraction digits into m and k, the
          // exponent's sign and digits.
          const uint32_t dg = b - 0x30;
          if (n == 1) {
            st.acc[3] |= 1u << 24;
          } else if ((n == 2 || n == 3) && (s == 0 || s == 1 || s == 3)) {
            const uint64_t m = (uint64_t)st.acc[0] | ((uint64_t)st.acc[1] << 32);
            if (m < kMantissaCap) {
              const uint64_t m2 = m * 10 + dg;
              st.acc[0] = (uint32_t)m2;
              st.acc[1] = (uint32_t)(m2 >> 32);
            } else {
              if ((int32_t)st.acc[2] < (1 << 20)) st.acc[2] += 1;
              if (dg) st.acc[3] |= 1u << 26;
            }
          } else if (n == 5) {
            const uint64_t m = (uint64_t)st.acc[0] | ((uint64_t)st.acc[1] << 32);
            if (m < kMantissaCap) {
              const uint64_t m2 = m * 10 + dg;
              st.acc[0] = (uint32_t)m2;
              st.acc[1] = (uint32_t)(m2 >> 32);
              if ((int32_t)st.acc[2] > -(1 << 20)) st.acc[2] -= 1;
            } else if (dg) {
              st.acc[3] |= 1u << 26;
            }
          } else if (n == 7 || n == 11) {
            if (b == 0x2D) st.acc[3] |= 1u << 25;
          } else if (n == 8 || n == 12) {
            uint32_t e = (st.acc[3] & 0xFFFFFFu) * 10 + dg;
            if (e > 999999) e = 999999;
            st.acc[3] = (st.acc[3] & ~0xFFFFFFu) | e;
          }
          return rOk;
        }
        if (!(s == 2 || s == 3 || s == 5 || s == 8)) return rReject;
        const uint32_t flags = f[0] >> 16, nf = nd_flags(P, f[1]);
        // Number(text) must be finite and meet the schema.  Without an
        // exponent, with at most 308 integer digits and no checks it is;
        // otherwise the value in the fast path decides, and a value outside
        // it is the host's.
        if ((flags & 1) || f[3] > 308 || (nf & (fNumCheck | fIntOnly))) {
          double v;
          if (!number_value(st.acc, &v)) return rUndecided;
          const int r = number_checks(P, f[1], nf, v);
          if (r != rOk) return r;
        }
        if (finish(st, vNumber) != rOk) return rReject;
        continue;
      }
      case kLiteral: {
        const char* lit = f[1] == 0 ? "true" : (f[1] == 1 ? "false" : "null");
        const uint32_t len = f[1] == 1 ? 5 : 4;
        if (f[1] > 2 || f[3] >= len || b != (uint32_t)(uint8_t)lit[f[3]]) return rReject;
        f[3] += 1;
        if (f[3] == len) return finish(st, f[1] == 2 ? vNull : vBoolean) == rOk ? rOk : rReject;
        return rOk;
      }
      case kChoice: {
        const uint32_t* v = P.values + f[1] * 4;
        uint32_t cont = 0, done = 0xFFFFFFFFu;
        for (uint32_t i = 0; i < v[2] && i < 32; ++i) {
          if (!((f[2] >> i) & 1)) continue;
          const uint32_t* c = P.cands + (v[1] + i) * 4;
          if (f[3] < c[1] && P.bytes[c[0] + f[3]] == b) cont |= 1u << i;
          if (f[3] == c[1] && done == 0xFFFFFFFFu) done = i;
        }
        if (cont) {
          f[2] = cont;
          f[3] += 1;
          return rOk;
        }
        if (done == 0xFFFFFFFFu) return rReject;
        if (finish(st, P.cands[(v[1] + done) * 4 + 2]) != rOk) return rReject;
        continue;
      }
      case kArray: {
        const uint32_t* nd = P.nodes + f[1] * kNodeWords;
        const uint32_t ph = fphase(f), minimum = nd[2], maximum = nd[3];
        if (ph == 0) {
          if (b != 0x5B) return rReject;
          set_phase(f, 1);
          return rOk;
        }
        if (ph == 1) {
          if (b == 0x5D) {
            if (f[3] < minimum) return rReject;
            if (nd[1] & fValueCheck) return rUndecided;
            return finish(st, vArray) == rOk ? rOk : rReject;
          }
          if (f[3] >= maximum) return rReject;
          if (st.depth >= kMaxDepth) return rUndecided;
          set_phase(f, 2);
          uint32_t* g = st.fr[st.depth++];
          g[0] = kValue;
          g[1] = nd[4];
          g[2] = 0;
          g[3] = 0;
          continue;
        }
        if (ph == 3) {
          if (b == 0x2C && f[3] < maximum) {
            if (st.depth >= kMaxDepth) return rUndecided;
            set_phase(f, 2);
            uint32_t* g = st.fr[st.depth++];
            g[0] = kValue;
            g[1] = nd[4];
            g[2] = 0;
            g[3] = 0;
            return rOk;
          }
          if (b == 0x5D && f[3] >= minimum) {
            if (nd[1] & fValueCheck) return rUndecided;
            if (nd[1] & fUnique) {
              if (!(f[2] & kItemsHost)) return rUndecided;
              if (!(f[2] & kItemsUnique)) return rReject;
            }
            return finish(st, vArray) == rOk ? rOk : rReject;
          }
          return rReject;
        }
        return rReject;
      }
      case kObject: {
        const uint32_t* nd = P.nodes + f[1] * kNodeWords;
        const uint32_t ph = fphase(f), nprops = nd[5], required = nd[7];
        const uint32_t minimum = nd[8], maximum = nd[9], used = f[2];
        const uint32_t nused = __builtin_popcount(used);
        if (ph == 0) {
          if (b != 0x7B) return rReject;
          set_phase(f, 1);
          return rOk;
        }
        if (ph == 1 || ph == 2) {
          if (b == 0x7D && ph == 1) {
            if (nused < minimum || (required & ~used)) return rReject;
            if (nd[1] & fValueCheck) return rUndecided;
            return finish(st, vObject) == rOk ? rOk : rReject;
          }
          if (b != 0x22 || nused >= maximum) return rReject;
          const uint32_t all = nprops >= 32 ? 0xFFFFFFFFu : ((1u << nprops) - 1u);
          const uint32_t live = all & ~used;
          if (!live) return rReject;
          if (st.depth >= kMaxDepth) return rUndecided;
          set_phase(f, 3);
          uint32_t* g = st.fr[st.depth++];
          g[0] = kKey;
          g[1] = f[1];
          g[2] = live;
          g[3] = 0;
          return rOk;
        }
        if (ph == 4) {
          if (b != 0x3A || f[3] >= nprops) return rReject;
          if (st.depth >= kMaxDepth) return rUndecided;
          set_phase(f, 5);
          const uint32_t* pr = P.props + (nd[6] + f[3]) * 4;
          uint32_t* g = st.fr[st.depth++];
          g[0] = kValue;
          g[1] = pr[2];
          g[2] = 0;
          g[3] = 0;
          return rOk;
        }
        if (ph == 6) {
          if (b == 0x2C && nused < maximum) {
            set_phase(f, 2);
            return rOk;
          }
          if (b == 0x7D && nused >= minimum && !(required & ~used)) {
            if (nd[1] & fValueCheck) return rUndecided;
            return finish(st, vObject) == rOk ? rOk : rReject;
          }
          return rReject;
        }
        return rReject;
      }
      case kKey: {
        const uint32_t* nd = P.nodes + f[1] * kNodeWords;
        const uint32_t nprops = nd[5] < 32 ? nd[5] : 32;
        if (b == 0x22) {
          uint32_t done = 0xFFFFFFFFu;
          for (uint32_t i = 0; i < nprops; ++i)
            if (((f[2] >> i) & 1) && P.props[(nd[6] + i) * 4 + 1] == f[3]) {
              done = i;
              break;
            }
          if (done == 0xFFFFFFFFu) return rReject;
          st.depth -= 1;
          if (st.depth == 0) return rReject;
          uint32_t* parent = st.fr[st.depth - 1];
          if (fkind(parent) != kObject) return rReject;
          parent[3] = done;
          set_phase(parent, 4);
          return rOk;
        }
        uint32_t cont = 0;
        for (uint32_t i = 0; i < nprops; ++i) {
          if (!((f[2] >> i) & 1)) continue;
          const uint32_t* pr = P.props + (nd[6] + i) * 4;
          if (f[3] < pr[1] && P.bytes[pr[0] + f[3]] == b) cont |= 1u << i;
        }
        if (!cont) return rReject;
        f[2] = cont;
        f[3] += 1;
        return rOk;
      }
      default:
        return rReject;
    }
  }
  return rReject;
}

// The complete getter (grammar.ts:270-280) and the value kind it reports.
__device__ bool args_complete(const Program& P, const State& st, uint32_t* kind) {
  if (st.args_complete) {
    *kind = st.args_kind;
    return true;
  }
  if (st.depth == 1 && fkind(st.fr[0]) == kChoice && st.fr[0][1] < P.n_values) {
    const uint32_t* f = st.fr[0];
    const uint32_t* v = P.values + f[1] * 4;
    for (uint32_t i = 0; i < v[2] && i < 32; ++i)
      if (((f[2] >> i) & 1) && P.cands[(v[1] + i) * 4 + 1] == f[3]) {
        *kind = P.cands[(v[1] + i) * 4 + 2];
        return true;
      }
  }
  return false;
}

__constant__ const uint8_t kNameLiteral[8] = {'"', 'n', 'a', 'm', 'e', '"', ':', '"'};
__constant__ const uint8_t kArgsLiteral[13] = {',', '"', 'a', 'r', 'g', 'u', 'm', 'e',
                                               'n', 't', 's', '"', ':'};

// ToolCallGrammar.feedByte (grammar.ts:716-796).
__device__ int tool_byte(const Program& P, State& st, uint32_t b) {
  for (int retry = 0; retry < 8; ++retry) {
    switch (st.phase) {
      case pArrayOpen:
        if (b != 0x5B) return rReject;
        st.phase = pCallOpen;
        return rOk;
      case pCallOpen:
        if (b != 0x7B) return rReject;
        st.phase = pNameLiteral;
        st.lit = 0;
        return rOk;
      case pNameLiteral:
        if (st.lit >= 8 || b != kNameLiteral[st.lit]) return rReject;
        if (++st.lit == 8) {
          st.phase = pToolName;
          const uint32_t all = st.n_tools >= 32 ? 0xFFFFFFFFu : ((1u << st.n_tools) - 1u);
          st.name_live = all & ~st.used_tools;
          st.name_off = 0;
        }
        return rOk;
      case pToolName: {
        const uint32_t n = st.n_tools < 32 ? st.n_tools : 32;
        if (b == 0x22) {
          uint32_t done = 0xFFFFFFFFu;
          for (uint32_t i = 0; i < n; ++i)
            if (((st.name_live >> i) & 1) && P.tools[i * 4 + 1] == st.name_off) {
              done = i;
              break;
            }
          if (done == 0xFFFFFFFFu) return rReject;
          st.cur_tool = done;
          st.phase = pArgsLiteral;
          st.lit = 0;
          return rOk;
        }
        uint32_t cont = 0;
        for (uint32_t i = 0; i < n; ++i) {
          if (!((st.name_live >> i) & 1)) continue;
          const uint32_t* t = P.tools + i * 4;
          if (st.name_off < t[1] && P.bytes[t[0] + st.name_off] == b) cont |= 1u << i;
        }
        if (!cont) return rReject;
        st.name_live = cont;
        st.name_off += 1;
        return rOk;
      }
      case pArgsLiteral:
        if (st.lit >= 13 || b != kArgsLiteral[st.lit]) return rReject;
        if (++st.lit == 13) {
          if (st.cur_tool >= st.n_tools) return rReject;
          st.args_present = 1;
          st.args_complete = 0;
          st.depth = 1;
          st.fr[0][0] = kValue;
          st.fr[0][1] = P.tools[st.cur_tool * 4 + 2];
          st.fr[0][2] = 0;
          st.fr[0][3] = 0;
          st.phase = pArgs;
        }
        return rOk;
      case pArgs: {
        if (!st.args_present) return rReject;
        uint32_t kind;
        if (args_complete(P, st, &kind)) {
          st.phase = pCallClose;
          continue;
        }
        return json_byte(P, st, b);
      }
      case pCallClose: {
        if (b != 0x7D) return rReject;
        uint32_t kind = 0xFFFFFFFFu;
        if (st.cur_tool >= st.n_tools || !st.args_present || !args_complete(P, st, &kind) ||
            kind != vObject)
          return rReject;
        st.n_calls += 1;
        st.used_tools |= 1u << st.cur_tool;
        st.phase = pAfterCall;
        return rOk;
      }
      case pAfterCall:
        if (b == 0x5D) {
          st.phase = pDone;
          return rOk;
        }
        if (b == 0x2C && st.n_calls < st.max_calls &&
            (uint32_t)__builtin_popcount(st.used_tools) < st.n_tools) {
          st.phase = pCallOpen;
          return rOk;
        }
        return rReject;
      default:
        return rReject;
    }
  }
  return rReject;
}

// One thread per token id: eligible pieces within the output limit are fed
// to a private copy of the state.  allowed / undecided: bit t of word t/32.
__global__ __launch_bounds__(kGThreads) void grammar_mask_kernel(
    Program P, const uint32_t* __restrict__ state, const uint32_t* __restrict__ offsets,
    const uint8_t* __restrict__ bytes, const uint8_t* __restrict__ eligible, uint32_t vocab,
    uint32_t budget, uint32_t* __restrict__ allowed, uint32_t* __restrict__ undecided) {
  const uint32_t tok = blockIdx.x * kGThreads + threadIdx.x;
  int res = rReject;
  if (tok < vocab && eligible[tok]) {
    const uint32_t begin = offsets[tok], end = offsets[tok + 1];
    if (end > begin && end - begin <= budget) {
      State st;
      st.phase = state[0];
      st.lit = state[1];
      st.name_live = state[2];
      st.name_off = state[3];
      st.cur_tool = state[4];
      st.used_tools = state[5];
      st.n_calls = state[6];
      st.max_calls = state[7];
      st.n_tools = state[8] < P.n_tools ? state[8] : P.n_tools;
      st.args_present = state[9];
      st.args_complete = state[10];
      st.args_kind = state[11];
      st.depth = state[12] < kMaxDepth ? state[12] : kMaxDepth;
      for (int w = 0; w < 4; ++w) st.acc[w] = state[16 + w];
      for (uint32_t i = 0; i < st.depth; ++i)
        for (int w = 0; w < 4; ++w) st.fr[i][w] = state[24 + i * 4 + w];
      res = rOk;
      for (uint32_t i = begin; i < end && res == rOk; ++i) res = tool_byte(P, st, bytes[i]);
    }
  }
  const uint64_t ok = __ballot(res == rOk), und = __ballot(res == rUndecided);
  const uint32_t lane = threadIdx.x & 63, base = tok - lane;  // first token of the wave
  if (lane == 0 && base < vocab) {
    allowed[base / 32] = (uint32_t)ok;
    undecided[base / 32] = (uint32_t)und;
  }
  if (lane == 32 && base + 32 < vocab) {
    allowed[base / 32 + 1] = (uint32_t)(ok >> 32);
    undecided[base / 32 + 1] = (uint32_t)(und >> 32);
  }
}

}  // namespace

hipError_t nd_launch_grammar_mask(const nd_grammar* g, const uint32_t* state,
                                  const nd_pieces* pc, uint32_t budget, uint32_t* allowed,
                                  uint32_t* undecided, hipStream_t s) {
  Program P;
  P.nodes = g->words + g->off[0];
  P.values = g->words + g->off[1];
  P.alts = g->words + g->off[2];
  P.props = g->words + g->off[3];
  P.cands = g->words + g->off[4];
  P.tools = g->words + g->off[5];
  P.bytes = reinterpret_cast<const uint8_t*>(g->words) + g->bytes_off;
  P.regex = g->words + g->regex_off;
  P.n_nodes = g->n_nodes;
  P.n_values = g->n_values;
  P.n_tools = g->n_tools;
  const uint32_t blocks = (pc->vocab + kGThreads - 1) / kGThreads;
  hipLaunchKernelGGL(grammar_mask_kernel, dim3(blocks), dim3(kGThreads), 0, s, P, state,
                     pc->offsets, pc->bytes, pc->eligible, pc->vocab, budget, allowed, undecided);
  return hipGetLastError();
}

// ------------------------------------------------------------------ C ABI

namespace {

constexpr uint32_t kGrammarMagic = 0x4E444752u;  // "RGDN"
constexpr uint32_t kStateHeaderWords = 24;

// Every table reference inside the program stays inside the program, so that
// the kernel's reads are in bounds for any state whose own indices it checks.
const char* check_program(const uint32_t* w, uint32_t n, nd_grammar* g) {
  if (n < 16 || w[0] != kGrammarMagic) return "bad magic or header";
  const uint32_t counts[6] = {w[1], w[3], w[5], w[7], w[9], w[11]};
  const uint32_t widths[6] = {kNodeWords, 4, 1, 4, 4, 4};
  for (int i = 0; i < 6; ++i) {
    const uint64_t end = (uint64_t)w[2 + 2 * i] + (uint64_t)counts[i] * widths[i];
    if (w[2 + 2 * i] < 16 || end > n) return "table outside the program";
    g->off[i] = w[2 + 2 * i];
  }
  const uint64_t bytes_end = (uint64_t)w[13] + w[14];
  if (w[13] < 64 || bytes_end > (uint64_t)n * 4) return "bytes outside the program";
  g->bytes_off = w[13];
  // Pattern automata: the words from w[15] up to the bytes.
  uint32_t rx_len = 0;
  if (w[15]) {
    if (w[15] < 16 || w[15] > w[13] / 4) return "pattern automata outside the program";
    rx_len = w[13] / 4 - w[15];
  }
  g->regex_off = w[15];
  auto regex_ok = [&](uint32_t entry) {
    if ((uint64_t)entry + 4 > rx_len) return false;
    const uint32_t* r = w + w[15] + entry;
    const uint64_t ns = r[0], nc = r[1], nb = r[2];
    if (ns == 0 || nc == 0 || nb == 0 || ns > 1024 || nc > 65536) return false;
    if (entry + 4 + nb + ns + ns * nc > rx_len || (r[4] & 0xFFFFu) != 0) return false;
    for (uint64_t i = 0; i < nb; ++i)
      if ((r[4 + i] >> 16) >= nc || (i && (r[4 + i] & 0xFFFFu) <= (r[3 + i] & 0xFFFFu)))
        return false;
    const uint32_t* t = r + 4 + nb + ns;
    for (uint64_t i = 0; i < ns * nc; ++i)
      if (t[i] >= ns) return false;
    return true;
  };
  g->n_nodes = counts[0];
  g->n_values = counts[1];
  g->n_tools = counts[5];
  if (g->n_tools == 0 || g->n_tools > 32) return "1..32 tools";
  const uint32_t *nodes = w + g->off[0], *values = w + g->off[1], *alts = w + g->off[2],
                 *props = w + g->off[3], *cands = w + g->off[4], *tools = w + g->off[5];
  auto bytes_ok = [&](uint32_t first, uint32_t len) {
    return (uint64_t)first + len <= w[14];
  };
  for (uint32_t i = 0; i < counts[0]; ++i) {
    const uint32_t* nd = nodes + i * kNodeWords;
    if (nd[4] >= counts[1] || nd[5] > 32 || (uint64_t)nd[6] + nd[5] > counts[3])
      return "node references outside the tables";
    if ((nd[15] && !regex_ok(nd[15] - 1)) || ((nd[12] & kcPattern) && !nd[15]))
      return "pattern automaton outside the table";
  }
  for (uint32_t i = 0; i < counts[1]; ++i) {
    const uint32_t* v = values + i * 4;
    if (v[0] == 0 && (uint64_t)v[1] + v[2] > counts[2]) return "alternatives outside";
    if (v[0] == 1 && (v[2] > 32 || (uint64_t)v[1] + v[2] > counts[4])) return "candidates outside";
    if (v[0] > 2) return "bad value kind";
  }
  for (uint32_t i = 0; i < counts[2]; ++i)
    if (alts[i] >= counts[0]) return "alternative node outside";
  for (uint32_t i = 0; i < counts[3]; ++i)
    if (!bytes_ok(props[i * 4], props[i * 4 + 1]) || props[i * 4 + 2] >= counts[1])
      return "property outside";
  for (uint32_t i = 0; i < counts[4]; ++i)
    if (!bytes_ok(cands[i * 4], cands[i * 4 + 1]) || cands[i * 4 + 2] > 5) return "candidate outside";
  for (uint32_t i = 0; i < counts[5]; ++i)
    if (!bytes_ok(tools[i * 4], tools[i * 4 + 1]) || tools[i * 4 + 2] >= counts[1])
      return "tool outside";
  return nullptr;
}

}  // namespace

nd_status nd_check_grammar_state(nd_ctx* ctx, const uint32_t* state, uint32_t n_state_words) {
  if (n_state_words < kStateHeaderWords || state[12] > 24 ||
      n_state_words < kStateHeaderWords + 4 * state[12])
    return nd_fail(ctx, n_state_words >= kStateHeaderWords && state[12] > 24 ? ND_ERR_UNSUPPORTED
                                                                              : ND_ERR_INVALID,
                   "grammar state of %u words with depth %u (at most 24 frames)", n_state_words,
                   n_state_words >= kStateHeaderWords ? state[12] : 0);
  return ND_OK;
}

extern "C" {

nd_status nd_pieces_upload(nd_ctx* ctx, const uint32_t* offsets, const uint8_t* bytes,
                           const uint8_t* eligible, uint32_t vocab, nd_pieces** out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!offsets || !eligible || !out || vocab == 0 || (offsets[vocab] && !bytes))
    return nd_fail(ctx, ND_ERR_INVALID, "nd_pieces_upload: NULL argument or empty vocabulary");
  *out = nullptr;
  for (uint32_t i = 0; i < vocab; ++i)
    if (offsets[i + 1] < offsets[i])
      return nd_fail(ctx, ND_ERR_INVALID, "piece offsets must not decrease (token %u)", i);
  const size_t ob = ((size_t)(vocab + 1) * 4 + 255) & ~size_t(255);
  const size_t eb = ((size_t)vocab + 255) & ~size_t(255);
  const size_t bb = offsets[vocab];
  ND_HIP(ctx, hipSetDevice(ctx->device));
  nd_pieces* pc = new nd_pieces();
  char* base = nullptr;
  hipError_t e = hipMalloc(&base, ob + eb + bb + 1);
  if (e == hipSuccess) {
    pc->offsets = reinterpret_cast<uint32_t*>(base);
    pc->eligible = reinterpret_cast<uint8_t*>(base + ob);
    pc->bytes = reinterpret_cast<uint8_t*>(base + ob + eb);
    pc->vocab = vocab;
    e = hipMemcpyAsync(pc->offsets, offsets, (size_t)(vocab + 1) * 4, hipMemcpyHostToDevice,
                       ctx->stream);
  }
  if (e == hipSuccess)
    e = hipMemcpyAsync(pc->eligible, eligible, vocab, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess && bb)
    e = hipMemcpyAsync(pc->bytes, bytes, bb, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    hipFree(base);
    delete pc;
    return nd_hip_fail(ctx, e, "piece upload");
  }
  ctx->pieces.insert(pc);
  *out = pc;
  return ND_OK;
}

nd_status nd_pieces_free(nd_ctx* ctx, nd_pieces* pc) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!pc) return ND_OK;
  if (!ctx->pieces.erase(pc)) return nd_fail(ctx, ND_ERR_INVALID, "pieces do not belong to context");
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  hipFree(pc->offsets);
  delete pc;
  return ND_OK;
}

nd_status nd_grammar_upload(nd_ctx* ctx, const uint32_t* program, uint32_t n_words,
                            nd_grammar** out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!program || !out) return nd_fail(ctx, ND_ERR_INVALID, "nd_grammar_upload: NULL argument");
  *out = nullptr;
  nd_grammar* g = new nd_grammar();
  if (const char* why = check_program(program, n_words, g)) {
    delete g;
    return nd_fail(ctx, ND_ERR_INVALID, "grammar program rejected: %s", why);
  }
  ND_HIP(ctx, hipSetDevice(ctx->device));
  hipError_t e = hipMalloc(&g->words, (size_t)n_words * 4);
  if (e == hipSuccess)
    e = hipMemcpyAsync(g->words, program, (size_t)n_words * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    hipFree(g->words);
    delete g;
    return nd_hip_fail(ctx, e, "grammar upload");
  }
  ctx->grammars.insert(g);
  *out = g;
  return ND_OK;
}

nd_status nd_grammar_free(nd_ctx* ctx, nd_grammar* g) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!g) return ND_OK;
  if (!ctx->grammars.erase(g)) return nd_fail(ctx, ND_ERR_INVALID, "grammar does not belong to context");
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  hipFree(g->words);
  delete g;
  return ND_OK;
}

nd_status nd_grammar_mask_d(nd_ctx* ctx, const nd_grammar* g, const uint32_t* state_dev,
                            const nd_pieces* pc, uint32_t budget, uint32_t* allowed_dev,
                            uint32_t* undecided_dev, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!g || !pc || !state_dev || !allowed_dev || !undecided_dev)
    return nd_fail(ctx, ND_ERR_INVALID, "nd_grammar_mask_d: NULL argument");
  ND_HIP(ctx, nd_launch_grammar_mask(g, state_dev, pc, budget, allowed_dev, undecided_dev,
                                     nd_pick_stream(ctx, stream)));
  return ND_OK;
}

nd_status nd_grammar_mask(nd_ctx* ctx, const nd_grammar* g, const uint32_t* state,
                          uint32_t n_state_words, const nd_pieces* pc, uint32_t budget,
                          uint32_t* allowed, uint32_t* undecided) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!g || !pc || !state || !allowed || !undecided)
    return nd_fail(ctx, ND_ERR_INVALID, "nd_grammar_mask: NULL argument");
  nd_status st = nd_check_grammar_state(ctx, state, n_state_words);
  if (st != ND_OK) return st;
  const size_t words = ((size_t)pc->vocab + 31) / 32;
  const size_t sb = ((size_t)n_state_words * 4 + 255) & ~size_t(255);
  if (!ctx->stage || ctx->stage_bytes < sb + 2 * words * 4) {
    // The staging buffer is shared with the other host-pointer calls.
    if (ctx->stage) {
      ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
      ND_HIP(ctx, hipFree(ctx->stage));
      ctx->stage = nullptr;
      ctx->stage_bytes = 0;
    }
    const size_t want = std::max<size_t>(sb + 2 * words * 4, 1u << 20);
    ND_HIP(ctx, hipMalloc(&ctx->stage, want));
    ctx->stage_bytes = want;
  }
  char* base = reinterpret_cast<char*>(ctx->stage);
  uint32_t* dstate = reinterpret_cast<uint32_t*>(base);
  uint32_t* dallowed = reinterpret_cast<uint32_t*>(base + sb);
  uint32_t* dund = dallowed + words;
  ND_HIP(ctx, hipMemcpyAsync(dstate, state, (size_t)n_state_words * 4, hipMemcpyHostToDevice,
                             ctx->stream));
  ND_HIP(ctx, nd_launch_grammar_mask(g, dstate, pc, budget, dallowed, dund, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(allowed, dallowed, words * 4, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(undecided, dund, words * 4, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

}  // extern "C"
