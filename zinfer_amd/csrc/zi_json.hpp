// JSON validator state machine (src/grammar.zig:59-443), shared by the host
// entry points (consume after a token is accepted, src/gen.zig:624) and the
// mask kernel (one lane per token piece).  The 64-entry container stack is a
// bit word: bit d set means stack[d] == .array.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "zinfer_hip.h"

namespace zi {

// State, EscapeState, NumState in declaration order (src/grammar.zig:13-57).
enum : uint32_t {
    kJStart, kJKeyOrClose, kJKeyOnly, kJInKey, kJColon, kJValue,
    kJArrValOrClose, kJInStr, kJInNum, kJInLit, kJCommaOrClose, kJFinished, kJStates
};
enum : uint32_t { kEscNone, kEscEscaped, kEscHex1, kEscHex2, kEscHex3, kEscHex4 };
enum : uint32_t { kNumMinus, kNumZero, kNumInt, kNumDot, kNumFrac, kNumExp, kNumExpSign, kNumExpDigits };
constexpr uint32_t kJsonMaxDepth = 64;  // JsonValidator.stack: [64]ContainerType
// Inside the machine, State.inside_num with NumState n is the one state
// kJNum + n, so that every transition writes a single state variable.
constexpr uint32_t kJNum = kJStates;

struct JsonFsm {
    uint64_t stack;
    uint64_t lit;  // lit_expected, byte i at bits 8i
    uint32_t state, escape, num, depth, lit_len, lit_idx, object_only;  // num: the last NumState

    __host__ __device__ static bool ws(uint32_t b) { return b == ' ' || b == '\t' || b == '\n' || b == '\r'; }
    __host__ __device__ static bool digit(uint32_t b) { return b - '0' < 10u; }
    __host__ __device__ static bool hex(uint32_t b) {  // isHex, :55-57
        return digit(b) || (b | 0x20u) - 'a' < 6u;
    }

    __host__ __device__ void load(const zi_json_state &s) {
        stack = s.stack;
        memcpy(&lit, s.lit_expected, 8);  // little-endian: byte i at bits 8i
        state = s.state == kJInNum ? kJNum + s.num : s.state;
        escape = s.escape;
        num = s.num;
        depth = s.depth;
        lit_len = s.lit_len;
        lit_idx = s.lit_idx;
        object_only = s.object_only;
    }
    __host__ __device__ void store(zi_json_state &s) const {
        s.stack = stack;
        memcpy(s.lit_expected, &lit, 8);
        s.state = (uint8_t)(state >= kJNum ? kJInNum : state);
        s.escape = (uint8_t)escape;
        s.num = (uint8_t)(state >= kJNum ? state - kJNum : num);
        s.depth = (uint8_t)depth;
        s.lit_len = (uint8_t)lit_len;
        s.lit_idx = (uint8_t)lit_idx;
        s.object_only = (uint8_t)object_only;
    }

    __host__ __device__ bool finished() const { return state == kJFinished && depth == 0; }  // :78-80

    __host__ __device__ bool push(bool array, uint32_t next) {
        if (depth >= kJsonMaxDepth) return false;
        const uint64_t bit = 1ull << depth;
        stack = array ? (stack | bit) : (stack & ~bit);
        depth += 1;
        state = next;
        return true;
    }
    __host__ __device__ bool top_is_array() const { return (stack >> (depth - 1)) & 1ull; }

    // stepString (:82-132): a \u escape ends after three hex digits (hex3
    // returns to none; hex4 is never entered).
    __host__ __device__ bool step_string(uint32_t b, uint32_t next) {
        switch (escape) {
        case kEscNone:
            if (b == '\\') { escape = kEscEscaped; return true; }
            if (b == '"') { state = next; return true; }
            return b >= 0x20;
        case kEscEscaped:
            if (b == '"' || b == '\\' || b == '/' || b == 'b' || b == 'f' || b == 'n' || b == 'r' || b == 't') {
                escape = kEscNone;
                return true;
            }
            if (b == 'u') { escape = kEscHex1; return true; }
            return false;
        case kEscHex1:
        case kEscHex2:
        case kEscHex3:
            if (!hex(b)) return false;
            escape = escape == kEscHex3 ? kEscNone : escape + 1;
            return true;
        default:
            return false;
        }
    }

    __host__ __device__ void literal(uint64_t word, uint32_t len) {
        lit = word;
        lit_len = len;
        lit_idx = 1;
        state = kJInLit;
    }

    // stepValueStart (:134-192)
    __host__ __device__ bool value_start(uint32_t b) {
        if (b == '"') { escape = kEscNone; state = kJInStr; return true; }
        if (b == '{') return push(false, kJKeyOrClose);
        if (b == '[') return push(true, kJArrValOrClose);
        if (b == '-') { state = kJNum + kNumMinus; return true; }
        if (b == '0') { state = kJNum + kNumZero; return true; }
        if (b - '1' < 9u) { state = kJNum + kNumInt; return true; }
        if (b == 't') { literal(0x65757274ull, 4); return true; }    // "true"
        if (b == 'f') { literal(0x65736c6166ull, 5); return true; }  // "false"
        if (b == 'n') { literal(0x6c6c756eull, 4); return true; }    // "null"
        return false;
    }

    // transitionComma (:398-408) / transitionClose (:410-425)
    __host__ __device__ bool comma() {
        if (depth == 0) return false;
        state = top_is_array() ? kJValue : kJKeyOnly;
        return true;
    }
    __host__ __device__ bool close(uint32_t b) {
        if (depth == 0) return false;
        if ((b == ']') != top_is_array()) return false;
        depth -= 1;
        state = depth == 0 ? kJFinished : kJCommaOrClose;
        return true;
    }
    // stepNumDelimiter (:383-396) from a NumState that canTerminate (:47-52):
    // the callers are the zero, int_digits, frac_digits and exp_digits states.
    __host__ __device__ bool num_delim(uint32_t b, uint32_t n) {
        num = n;  // the reference keeps num_state after the number ends
        if (ws(b)) { state = kJCommaOrClose; return true; }
        if (b == ',') return comma();
        if (b == '}' || b == ']') return close(b);
        return false;
    }

    // stepByte (:195-381)
    __host__ __device__ bool step(uint32_t b) {
        switch (state) {
        case kJStart:
            if (ws(b)) return true;
            if (b == '{') return push(false, kJKeyOrClose);
            if (!object_only && b == '[') return push(true, kJArrValOrClose);
            return false;
        case kJKeyOrClose:
            if (ws(b)) return true;
            if (b == '}') {  // the '{' just read is on the stack: depth >= 1
                if (depth == 0) return false;
                depth -= 1;
                state = depth == 0 ? kJFinished : kJCommaOrClose;
                return true;
            }
            if (b == '"') { escape = kEscNone; state = kJInKey; return true; }
            return false;
        case kJKeyOnly:
            if (ws(b)) return true;
            if (b == '"') { escape = kEscNone; state = kJInKey; return true; }
            return false;
        case kJInKey:
            return step_string(b, kJColon);
        case kJColon:
            if (ws(b)) return true;
            if (b == ':') { state = kJValue; return true; }
            return false;
        case kJArrValOrClose:
            if (ws(b)) return true;
            if (b == ']') {
                if (depth == 0) return false;
                depth -= 1;
                state = depth == 0 ? kJFinished : kJCommaOrClose;
                return true;
            }
            return value_start(b);
        case kJValue:
            if (ws(b)) return true;
            return value_start(b);
        case kJInStr:
            return step_string(b, kJCommaOrClose);
        case kJNum + kNumMinus:
            if (b == '0') { state = kJNum + kNumZero; return true; }
            if (b - '1' < 9u) { state = kJNum + kNumInt; return true; }
            return false;
        case kJNum + kNumZero:
            if (b == '.') { state = kJNum + kNumDot; return true; }
            if (b == 'e' || b == 'E') { state = kJNum + kNumExp; return true; }
            return num_delim(b, kNumZero);
        case kJNum + kNumInt:
            if (digit(b)) return true;
            if (b == '.') { state = kJNum + kNumDot; return true; }
            if (b == 'e' || b == 'E') { state = kJNum + kNumExp; return true; }
            return num_delim(b, kNumInt);
        case kJNum + kNumDot:
            if (digit(b)) { state = kJNum + kNumFrac; return true; }
            return false;
        case kJNum + kNumFrac:
            if (digit(b)) return true;
            if (b == 'e' || b == 'E') { state = kJNum + kNumExp; return true; }
            return num_delim(b, kNumFrac);
        case kJNum + kNumExp:
            if (b == '+' || b == '-') { state = kJNum + kNumExpSign; return true; }
            if (digit(b)) { state = kJNum + kNumExpDigits; return true; }
            return false;
        case kJNum + kNumExpSign:
            if (digit(b)) { state = kJNum + kNumExpDigits; return true; }
            return false;
        case kJNum + kNumExpDigits:
            if (digit(b)) return true;
            return num_delim(b, kNumExpDigits);
        case kJInLit:
            if (lit_idx < lit_len && b == ((lit >> (8 * lit_idx)) & 0xFFu)) {
                lit_idx += 1;
                if (lit_idx == lit_len) state = kJCommaOrClose;
                return true;
            }
            return false;
        case kJCommaOrClose:
            if (ws(b)) return true;
            if (b == ',') return comma();
            if (b == '}' || b == ']') return close(b);
            return false;
        case kJFinished:
            return ws(b);
        default:
            return false;
        }
    }
};

// The state fields a piece can read, with the rest cleared: two states with
// the same canonical form give the same mask.
__host__ __device__ inline zi_json_state json_canonical(const zi_json_state &s) {
    zi_json_state c{};
    c.state = s.state;
    c.depth = s.depth;
    c.object_only = s.object_only;
    c.stack = s.depth >= 64 ? s.stack : (s.stack & ((1ull << s.depth) - 1ull));
    if (s.state == kJInKey || s.state == kJInStr) c.escape = s.escape;
    if (s.state == kJInNum) c.num = s.num;
    if (s.state == kJInLit) {
        c.lit_len = s.lit_len;
        c.lit_idx = s.lit_idx;
        for (int i = 0; i < 8; ++i) c.lit_expected[i] = s.lit_expected[i];
    }
    return c;
}


// ------------------------------------------------------------ table form
// The finite part of the machine as one flat state (37 of them) and a
// transition table over byte classes; the stack effects are six actions.
// The table is derived from JsonFsm::step (json_build_tables) and checked
// against it for every state, byte and stack shape before first use.
enum : uint32_t {
    kFStartObj, kFStartAny, kFKeyOrClose, kFKeyOnly, kFColon, kFValue, kFArrValOrClose, kFCommaOrClose,
    kFFinished,
    kFKey = 9,    // + EscapeState none..hex3
    kFStr = 14,   // + EscapeState none..hex3
    kFNum = 19,   // + NumState
    kFLit = 27,   // true idx 1-3, false idx 1-4, null idx 1-3
    kFCount = 37
};
enum : uint32_t { kAFail = 0x80, kAPushObj, kAPushArr, kAPop, kACloseObj, kACloseArr, kAComma };
constexpr int kClsStride = 64;  // table row stride (byte classes per state <= 64)

struct JsonTables {
    uint8_t cls[256];                  // byte -> class
    uint8_t tab[kFCount * kClsStride];  // flat state x class -> next flat state, or an action
};

constexpr uint64_t kLitTrue = 0x65757274ull, kLitFalse = 0x65736c6166ull, kLitNull = 0x6c6c756eull;

// The flat state of a machine state, or -1 when it has none (a literal other
// than true / false / null, or the unreachable hex4).
__host__ __device__ inline int json_flat(const JsonFsm &f) {
    switch (f.state) {
    case kJStart: return f.object_only ? kFStartObj : kFStartAny;
    case kJKeyOrClose: return kFKeyOrClose;
    case kJKeyOnly: return kFKeyOnly;
    case kJColon: return kFColon;
    case kJValue: return kFValue;
    case kJArrValOrClose: return kFArrValOrClose;
    case kJCommaOrClose: return kFCommaOrClose;
    case kJFinished: return kFFinished;
    case kJInKey: return f.escape <= kEscHex3 ? (int)(kFKey + f.escape) : -1;
    case kJInStr: return f.escape <= kEscHex3 ? (int)(kFStr + f.escape) : -1;
    case kJInLit: {
        const uint64_t m = f.lit_len >= 8 ? ~0ull : ((1ull << (8 * f.lit_len)) - 1ull);
        const uint64_t w = f.lit & m;
        if (f.lit_idx < 1 || f.lit_idx >= f.lit_len) return -1;
        if (w == kLitTrue && f.lit_len == 4) return kFLit + f.lit_idx - 1;
        if (w == kLitFalse && f.lit_len == 5) return kFLit + 3 + f.lit_idx - 1;
        if (w == kLitNull && f.lit_len == 4) return kFLit + 7 + f.lit_idx - 1;
        return -1;
    }
    default:
        return f.state >= kJNum && f.state < kJNum + 8 ? (int)(kFNum + (f.state - kJNum)) : -1;
    }
}

// A machine state for a flat state (escape / number / literal fields set).
__host__ __device__ inline JsonFsm json_unflat(uint32_t fl, uint32_t depth, uint64_t stack) {
    JsonFsm f{};
    f.stack = stack;
    f.depth = depth;
    f.object_only = fl != kFStartAny;
    f.num = kNumZero;
    f.escape = kEscNone;
    if (fl <= kFStartAny) f.state = kJStart;
    else if (fl < kFKey) {
        const uint32_t m[] = {kJStart, kJStart, kJKeyOrClose, kJKeyOnly, kJColon, kJValue, kJArrValOrClose,
                              kJCommaOrClose, kJFinished};
        f.state = m[fl];
    } else if (fl < kFStr) { f.state = kJInKey; f.escape = fl - kFKey; }
    else if (fl < kFNum) { f.state = kJInStr; f.escape = fl - kFStr; }
    else if (fl < kFLit) { f.state = kJNum + (fl - kFNum); f.num = fl - kFNum; }
    else {
        const uint32_t k = fl - kFLit;
        f.state = kJInLit;
        if (k < 3) { f.lit = kLitTrue; f.lit_len = 4; f.lit_idx = k + 1; }
        else if (k < 7) { f.lit = kLitFalse; f.lit_len = 5; f.lit_idx = k - 2; }
        else { f.lit = kLitNull; f.lit_len = 4; f.lit_idx = k - 6; }
    }
    return f;
}

// One byte class through the table form.  fl / depth / stack are updated
// only when the byte is accepted, as JsonFsm::step updates its fields.
__host__ __device__ inline bool json_class_step(const uint8_t *tab, uint32_t &fl, uint32_t &depth, uint64_t &stack,
                                                uint32_t c) {
    const uint32_t e = tab[fl * kClsStride + c];
    if (e < kAFail) {
        fl = e;
        return true;
    }
    if (e == kAFail) return false;
    if (e == kAPushObj || e == kAPushArr) {
        if (depth >= kJsonMaxDepth) return false;
        const uint64_t bit = 1ull << depth;
        stack = e == kAPushArr ? (stack | bit) : (stack & ~bit);
        depth += 1;
        fl = e == kAPushArr ? kFArrValOrClose : kFKeyOrClose;
        return true;
    }
    if (depth == 0) return false;
    const bool top_arr = (stack >> (depth - 1)) & 1ull;
    if (e == kAComma) {
        fl = top_arr ? kFValue : kFKeyOnly;
        return true;
    }
    if ((e == kACloseObj && top_arr) || (e == kACloseArr && !top_arr)) return false;
    depth -= 1;  // kAPop, or a close that matches the top
    fl = depth == 0 ? kFFinished : kFCommaOrClose;
    return true;
}

// The same step on a byte (class lookup first).
__host__ __device__ inline bool json_table_step(const uint8_t *cls, const uint8_t *tab, uint32_t &fl,
                                                uint32_t &depth, uint64_t &stack, uint32_t b) {
    return json_class_step(tab, fl, depth, stack, cls[b]);
}

// Builds the table from JsonFsm::step and checks the table form against it
// for every flat state, byte and stack shape.  Host only; false if they
// disagree anywhere.
inline bool json_build_tables(JsonTables &t) {
    static uint8_t full[kFCount][256];
    for (uint32_t fl = 0; fl < kFCount; ++fl)
        for (uint32_t b = 0; b < 256; ++b) {
            JsonFsm o = json_unflat(fl, 1, 0ull), a = json_unflat(fl, 1, 1ull);  // top .object / .array
            const bool ok_o = o.step(b), ok_a = a.step(b);
            uint32_t e;
            if (!ok_o && !ok_a) e = kAFail;
            else if (ok_o && ok_a && o.depth == 2 && a.depth == 2) e = ((o.stack >> 1) & 1ull) ? kAPushArr : kAPushObj;
            else if (ok_o && ok_a && o.depth == 0 && a.depth == 0) e = kAPop;
            else if (ok_o && !ok_a && o.depth == 0) e = kACloseObj;
            else if (!ok_o && ok_a && a.depth == 0) e = kACloseArr;
            else if (ok_o && ok_a && o.depth == 1 && a.depth == 1) {
                const int fo = json_flat(o), fa = json_flat(a);
                if (fo < 0 || fa < 0) return false;
                if (fo == fa) e = (uint32_t)fo;
                else if (fo == (int)kFKeyOnly && fa == (int)kFValue) e = kAComma;
                else return false;
            } else {
                return false;
            }
            full[fl][b] = (uint8_t)e;
        }
    // byte classes: bytes with the same column share a class
    int ncls = 0;
    uint32_t rep[256];
    for (uint32_t b = 0; b < 256; ++b) {
        int c = -1;
        for (int k = 0; k < ncls && c < 0; ++k) {
            bool same = true;
            for (uint32_t fl = 0; fl < kFCount && same; ++fl) same = full[fl][rep[k]] == full[fl][b];
            if (same) c = k;
        }
        if (c < 0) {
            if (ncls == kClsStride) return false;
            rep[ncls] = b;
            c = ncls++;
        }
        t.cls[b] = (uint8_t)c;
    }
    for (uint32_t fl = 0; fl < kFCount; ++fl)
        for (int c = 0; c < kClsStride; ++c) t.tab[fl * kClsStride + c] = c < ncls ? full[fl][rep[c]] : (uint8_t)kAFail;
    // check: table form == machine, every state x byte x stack shape
    const uint32_t depths[] = {0, 1, 1, 2, 2, 63, 64, 64};
    const uint64_t stacks[] = {0ull, 0ull, 1ull, 1ull, 2ull, 0x5555555555555555ull, ~0ull, 0ull};
    for (uint32_t fl = 0; fl < kFCount; ++fl)
        for (uint32_t b = 0; b < 256; ++b)
            for (int s = 0; s < 8; ++s) {
                JsonFsm m = json_unflat(fl, depths[s], stacks[s]);
                const bool ok = m.step(b);
                uint32_t f2 = fl, d2 = depths[s];
                uint64_t s2 = stacks[s];
                const bool ok2 = json_table_step(t.cls, t.tab, f2, d2, s2, b);
                if (ok != ok2) return false;
                if (!ok) continue;
                const uint64_t mask = d2 >= 64 ? ~0ull : ((1ull << d2) - 1ull);
                if ((int)f2 != json_flat(m) || d2 != m.depth || (s2 & mask) != (m.stack & mask)) return false;
            }
    return true;
}

}  // namespace zi
