/*
 * grammar_oracle.c -- CPU restatement of the reference's JSON validator and
 * its logit mask (src/grammar.zig).  TEST INFRASTRUCTURE ONLY: nothing in the
 * product links, loads or calls it.
 *
 * The state keeps the reference's shape (enum state, a 64-entry container
 * stack, escape / number / literal sub-states); the product packs the stack
 * into a bit word instead, so the two are written independently.
 */
#include <string.h>
#include <time.h>

#include "oracle.h"

/* State, EscapeState, NumState in declaration order, src/grammar.zig:13-57. */
enum { ST_START, ST_OBJ_KEY_OR_CLOSE, ST_OBJ_KEY_ONLY, ST_INSIDE_KEY, ST_OBJ_COLON, ST_EXPECT_VALUE,
       ST_ARR_VAL_OR_CLOSE, ST_INSIDE_STR, ST_INSIDE_NUM, ST_INSIDE_LIT, ST_COMMA_OR_CLOSE, ST_FINISHED };
enum { ESC_NONE, ESC_ESCAPED, ESC_HEX1, ESC_HEX2, ESC_HEX3, ESC_HEX4 };
enum { NUM_MINUS, NUM_ZERO, NUM_INT, NUM_DOT, NUM_FRAC, NUM_EXP, NUM_EXP_SIGN, NUM_EXP_DIGITS };
enum { CT_OBJECT = 0, CT_ARRAY = 1 };

static int is_ws(uint8_t b) { return b == ' ' || b == '\t' || b == '\n' || b == '\r'; }
static int is_digit(uint8_t b) { return b >= '0' && b <= '9'; }
/* isHex, src/grammar.zig:55-57 */
static int is_hex(uint8_t b) { return is_digit(b) || (b >= 'a' && b <= 'f') || (b >= 'A' && b <= 'F'); }

/* initObjectOnly / initAny, src/grammar.zig:70-76; field defaults :60-68. */
void or_json_init(or_json *j, int object_only) {
    memset(j, 0, sizeof *j);
    j->state = ST_START;
    j->escape = ESC_NONE;
    j->num = NUM_ZERO;
    j->object_only = object_only ? 1 : 0;
}

/* isFinished, src/grammar.zig:78-80 */
int or_json_is_finished(const or_json *j) { return j->state == ST_FINISHED && j->depth == 0; }

static int push(or_json *j, int ct, int next) {
    if (j->depth >= 64) return 0;
    j->stack[j->depth++] = (uint8_t)ct;
    j->state = next;
    return 1;
}

/* stepString, src/grammar.zig:82-132 (three hex digits end a \u escape:
 * hex3 returns to none, hex4 is never entered). */
static int step_string(or_json *j, uint8_t b, int next_state) {
    switch (j->escape) {
    case ESC_NONE:
        if (b == '\\') { j->escape = ESC_ESCAPED; return 1; }
        if (b == '"') { j->state = next_state; return 1; }
        return b >= 0x20;
    case ESC_ESCAPED:
        if (b == '"' || b == '\\' || b == '/' || b == 'b' || b == 'f' || b == 'n' || b == 'r' || b == 't') {
            j->escape = ESC_NONE;
            return 1;
        }
        if (b == 'u') { j->escape = ESC_HEX1; return 1; }
        return 0;
    case ESC_HEX1:
        if (is_hex(b)) { j->escape = ESC_HEX2; return 1; }
        return 0;
    case ESC_HEX2:
        if (is_hex(b)) { j->escape = ESC_HEX3; return 1; }
        return 0;
    case ESC_HEX3:
        if (is_hex(b)) { j->escape = ESC_NONE; return 1; }
        return 0;
    default:
        return 0;  /* hex4: unreachable in the reference */
    }
}

static void set_literal(or_json *j, const char *word) {
    const size_t n = strlen(word);
    memcpy(j->lit_expected, word, n);
    j->lit_len = (uint8_t)n;
    j->lit_idx = 1;
    j->state = ST_INSIDE_LIT;
}

/* stepValueStart, src/grammar.zig:134-192 */
static int step_value_start(or_json *j, uint8_t b) {
    if (b == '"') { j->escape = ESC_NONE; j->state = ST_INSIDE_STR; return 1; }
    if (b == '{') return push(j, CT_OBJECT, ST_OBJ_KEY_OR_CLOSE);
    if (b == '[') return push(j, CT_ARRAY, ST_ARR_VAL_OR_CLOSE);
    if (b == '-') { j->state = ST_INSIDE_NUM; j->num = NUM_MINUS; return 1; }
    if (b == '0') { j->state = ST_INSIDE_NUM; j->num = NUM_ZERO; return 1; }
    if (b >= '1' && b <= '9') { j->state = ST_INSIDE_NUM; j->num = NUM_INT; return 1; }
    if (b == 't') { set_literal(j, "true"); return 1; }
    if (b == 'f') { set_literal(j, "false"); return 1; }
    if (b == 'n') { set_literal(j, "null"); return 1; }
    return 0;
}

/* transitionComma, src/grammar.zig:398-408 */
static int transition_comma(or_json *j) {
    if (j->depth == 0) return 0;
    j->state = j->stack[j->depth - 1] == CT_OBJECT ? ST_OBJ_KEY_ONLY : ST_EXPECT_VALUE;
    return 1;
}

/* transitionClose, src/grammar.zig:410-425 */
static int transition_close(or_json *j, uint8_t b) {
    if (j->depth == 0) return 0;
    const int cur = j->stack[j->depth - 1];
    if ((b == '}' && cur == CT_OBJECT) || (b == ']' && cur == CT_ARRAY)) {
        j->depth -= 1;
        j->state = j->depth == 0 ? ST_FINISHED : ST_COMMA_OR_CLOSE;
        return 1;
    }
    return 0;
}

/* canTerminate, src/grammar.zig:47-52 */
static int num_can_terminate(int n) { return n == NUM_ZERO || n == NUM_INT || n == NUM_FRAC || n == NUM_EXP_DIGITS; }

/* stepNumDelimiter, src/grammar.zig:383-396 */
static int step_num_delimiter(or_json *j, uint8_t b) {
    if (!num_can_terminate(j->num)) return 0;
    if (is_ws(b)) { j->state = ST_COMMA_OR_CLOSE; return 1; }
    if (b == ',') return transition_comma(j);
    if (b == '}' || b == ']') return transition_close(j, b);
    return 0;
}

/* stepByte, src/grammar.zig:195-381 */
int or_json_step_byte(or_json *j, uint8_t b) {
    switch (j->state) {
    case ST_START:
        if (is_ws(b)) return 1;
        if (b == '{') return push(j, CT_OBJECT, ST_OBJ_KEY_OR_CLOSE);
        if (!j->object_only && b == '[') return push(j, CT_ARRAY, ST_ARR_VAL_OR_CLOSE);
        return 0;
    case ST_OBJ_KEY_OR_CLOSE:
        if (is_ws(b)) return 1;
        if (b == '}') {
            if (j->depth == 0) return 0;
            j->depth -= 1;
            j->state = j->depth == 0 ? ST_FINISHED : ST_COMMA_OR_CLOSE;
            return 1;
        }
        if (b == '"') { j->escape = ESC_NONE; j->state = ST_INSIDE_KEY; return 1; }
        return 0;
    case ST_OBJ_KEY_ONLY:
        if (is_ws(b)) return 1;
        if (b == '"') { j->escape = ESC_NONE; j->state = ST_INSIDE_KEY; return 1; }
        return 0;
    case ST_INSIDE_KEY:
        return step_string(j, b, ST_OBJ_COLON);
    case ST_OBJ_COLON:
        if (is_ws(b)) return 1;
        if (b == ':') { j->state = ST_EXPECT_VALUE; return 1; }
        return 0;
    case ST_ARR_VAL_OR_CLOSE:
        if (is_ws(b)) return 1;
        if (b == ']') {
            if (j->depth == 0) return 0;
            j->depth -= 1;
            j->state = j->depth == 0 ? ST_FINISHED : ST_COMMA_OR_CLOSE;
            return 1;
        }
        return step_value_start(j, b);
    case ST_EXPECT_VALUE:
        if (is_ws(b)) return 1;
        return step_value_start(j, b);
    case ST_INSIDE_STR:
        return step_string(j, b, ST_COMMA_OR_CLOSE);
    case ST_INSIDE_NUM:
        switch (j->num) {
        case NUM_MINUS:
            if (b == '0') { j->num = NUM_ZERO; return 1; }
            if (b >= '1' && b <= '9') { j->num = NUM_INT; return 1; }
            return 0;
        case NUM_ZERO:
            if (b == '.') { j->num = NUM_DOT; return 1; }
            if (b == 'e' || b == 'E') { j->num = NUM_EXP; return 1; }
            return step_num_delimiter(j, b);
        case NUM_INT:
            if (is_digit(b)) return 1;
            if (b == '.') { j->num = NUM_DOT; return 1; }
            if (b == 'e' || b == 'E') { j->num = NUM_EXP; return 1; }
            return step_num_delimiter(j, b);
        case NUM_DOT:
            if (is_digit(b)) { j->num = NUM_FRAC; return 1; }
            return 0;
        case NUM_FRAC:
            if (is_digit(b)) return 1;
            if (b == 'e' || b == 'E') { j->num = NUM_EXP; return 1; }
            return step_num_delimiter(j, b);
        case NUM_EXP:
            if (b == '+' || b == '-') { j->num = NUM_EXP_SIGN; return 1; }
            if (is_digit(b)) { j->num = NUM_EXP_DIGITS; return 1; }
            return 0;
        case NUM_EXP_SIGN:
            if (is_digit(b)) { j->num = NUM_EXP_DIGITS; return 1; }
            return 0;
        case NUM_EXP_DIGITS:
            if (is_digit(b)) return 1;
            return step_num_delimiter(j, b);
        default:
            return 0;
        }
    case ST_INSIDE_LIT:
        if (j->lit_idx < j->lit_len && b == j->lit_expected[j->lit_idx]) {
            j->lit_idx += 1;
            if (j->lit_idx == j->lit_len) j->state = ST_COMMA_OR_CLOSE;
            return 1;
        }
        return 0;
    case ST_COMMA_OR_CLOSE:
        if (is_ws(b)) return 1;
        if (b == ',') return transition_comma(j);
        if (b == '}' || b == ']') return transition_close(j, b);
        return 0;
    case ST_FINISHED:
        return is_ws(b);
    default:
        return 0;
    }
}

/* tryConsume, src/grammar.zig:428-434: a copy steps through the piece. */
int or_json_try_consume(const or_json *j, const uint8_t *piece, size_t n, or_json *out) {
    or_json c = *j;
    for (size_t i = 0; i < n; ++i)
        if (!or_json_step_byte(&c, piece[i])) return 0;
    if (out) *out = c;
    return 1;
}

/* consume, src/grammar.zig:437-443: in place; a failing byte leaves the
 * bytes before it applied. */
int or_json_consume(or_json *j, const uint8_t *piece, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!or_json_step_byte(j, piece[i])) return 0;
    return 1;
}

static int in_list(const uint32_t *ids, uint32_t n, uint32_t id) {
    for (uint32_t i = 0; i < n; ++i)
        if (ids[i] == id) return 1;
    return 0;
}

/* applyMask, src/grammar.zig:446-479, as the allowed-token bitmask: bit t of
 * out[t >> 5] is set when the reference leaves logit t unchanged.  eos < 0
 * means eos_id == null; eog lists Tokenizer.eog (isEog, src/tokenizer.zig:270). */
void or_json_mask(const or_json *j, const uint32_t *piece_off, const uint8_t *piece_buf, uint32_t V,
                  const uint32_t *eog, uint32_t n_eog, int64_t eos, uint32_t *out) {
    const int fin = or_json_is_finished(j);
    memset(out, 0, sizeof(uint32_t) * ((V + 31) / 32));
    for (uint32_t id = 0; id < V; ++id) {
        const uint8_t *p = piece_buf + piece_off[id];
        const size_t n = piece_off[id + 1] - piece_off[id];
        const int is_eos = eos >= 0 && (int64_t)id == eos;
        int keep;
        if (fin) {
            if (is_eos || in_list(eog, n_eog, id)) {
                keep = 1;
            } else {
                keep = n > 0;
                for (size_t i = 0; i < n && keep; ++i) keep = is_ws(p[i]);
            }
        } else if (in_list(eog, n_eog, id) || is_eos) {
            keep = 0;
        } else if (n == 0) {
            keep = 1;
        } else {
            keep = or_json_try_consume(j, p, n, NULL);
        }
        if (keep) out[id >> 5] |= 1u << (id & 31);
    }
}

/* The masks of `rows` states, repeated `reps` times; returns seconds. */
double or_bench_json_mask(const or_json *states, uint32_t rows, const uint32_t *piece_off,
                          const uint8_t *piece_buf, uint32_t V, const uint32_t *eog, uint32_t n_eog,
                          int64_t eos, uint32_t *out, uint32_t reps) {
    struct timespec a, b;
    const uint32_t W = (V + 31) / 32;
    clock_gettime(CLOCK_MONOTONIC, &a);
    for (uint32_t r = 0; r < reps; ++r)
        for (uint32_t i = 0; i < rows; ++i)
            or_json_mask(&states[i], piece_off, piece_buf, V, eog, n_eog, eos, out + (size_t)i * W);
    clock_gettime(CLOCK_MONOTONIC, &b);
    return (double)(b.tv_sec - a.tv_sec) + 1e-9 * (double)(b.tv_nsec - a.tv_nsec);
}
