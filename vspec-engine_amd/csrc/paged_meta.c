/*
 * paged_meta.c -- host bookkeeping of the paged KV cache.
 *
 * Policy of the reference allocator, kv_paged_cache.c, with the caps lifted:
 *   - sessions live in a fixed table of max_sessions slots, found by linear scan;
 *   - pages are allocated first-fit (lowest free index); on exhaustion the
 *     least-recently-touched session other than the requester is released whole and
 *     the scan retried (:90-122);
 *   - a page is freed when its reference count drops to zero (:37-59);
 *   - prefix reuse shares whole source pages into an empty target while the
 *     cumulative used count stays within max_tokens (:185-241); an append opens a
 *     new page when the last page is full or shared (:268-290);
 *   - a monotonically increasing clock stamps sessions and pages (:264-266).
 */
#include <stdlib.h>
#include <string.h>

#include "vspec_rocm_paged.h"

typedef struct Page {
    uint8_t allocated;
    uint32_t owner_slot;
    uint32_t used_tokens;
    uint32_t ref_count;
    uint64_t last_touch_step;
} Page;

typedef struct Session {
    uint8_t active;
    uint64_t session_id;
    uint64_t last_touch_step;
    uint64_t gen; /* stamp of this activation of the slot (0 while free) */
    size_t total_tokens;
    size_t page_count;
    uint32_t* pages; /* max_pages_per_session entries */
} Session;

/* What vspec_rocm_paged_plan_step_update last wrote into one row of the caller's tables:
 * the entries [0, len) of session `slot` in its activation `gen`, -1 / 0 after them. */
typedef struct RowState {
    uint32_t slot;
    uint32_t len;
    uint64_t gen;
} RowState;

struct VspecRocmPagedMeta {
    size_t page_tokens;
    size_t max_pages;
    size_t max_sessions;
    size_t max_pages_per_session;
    VspecRocmPagedStats stats;
    Page* page;
    Session* session;
    uint32_t* page_lists;
    uint64_t clock_step;
    uint64_t gen_clock;
    /* every page below it is allocated: the first-fit scan starts here */
    size_t free_hint;
    /* the tables plan_step_update writes (rows known only while these stay the same) */
    int32_t* rows_tables;
    int32_t* rows_used;
    size_t rows_max_blocks;
    size_t rows_cap;
    RowState* rows;
    /* per-call scratch of the planner, grown on demand */
    size_t scratch_cap;
    uint64_t* scratch_ids;
    int* scratch_slot;
    uint64_t* scratch_gen;
};

static int find_session(const VspecRocmPagedMeta* m, uint64_t id) {
    if (!m || id == 0u) return -1;
    for (size_t i = 0; i < m->max_sessions; ++i) {
        if (m->session[i].active && m->session[i].session_id == id) return (int)i;
    }
    return -1;
}

static int find_free_session(const VspecRocmPagedMeta* m) {
    for (size_t i = 0; i < m->max_sessions; ++i) {
        if (!m->session[i].active) return (int)i;
    }
    return -1;
}

static void release_session(VspecRocmPagedMeta* m, int slot) {
    Session* s = &m->session[slot];
    for (size_t i = 0; i < s->page_count; ++i) {
        const uint32_t p = s->pages[i];
        if (p >= m->max_pages) continue;
        if (m->page[p].ref_count > 0u) m->page[p].ref_count -= 1u;
        if (m->page[p].ref_count == 0u) {
            m->page[p].allocated = 0u;
            m->page[p].owner_slot = 0u;
            m->page[p].used_tokens = 0u;
            if (p < m->free_hint) m->free_hint = p;
        }
    }
    uint32_t* keep = s->pages;
    memset(s, 0, sizeof(*s));
    s->pages = keep;
}

static int evict_lru(VspecRocmPagedMeta* m, int protect) {
    int victim = -1;
    uint64_t oldest = UINT64_MAX;
    for (size_t i = 0; i < m->max_sessions; ++i) {
        if (!m->session[i].active || (int)i == protect) continue;
        if (m->session[i].last_touch_step < oldest) {
            oldest = m->session[i].last_touch_step;
            victim = (int)i;
        }
    }
    if (victim < 0) return 0;
    release_session(m, victim);
    m->stats.evict_session_count += 1u;
    return 1;
}

static long take_first_free(VspecRocmPagedMeta* m, int owner) {
    for (size_t i = m->free_hint; i < m->max_pages; ++i) {
        m->free_hint = i;
        if (!m->page[i].allocated) {
            Page* p = &m->page[i];
            p->allocated = 1u;
            p->owner_slot = (uint32_t)owner;
            p->used_tokens = 0u;
            p->ref_count = 1u;
            p->last_touch_step = m->clock_step;
            m->stats.page_alloc_count += 1u;
            m->free_hint = i + 1u;
            return (long)i;
        }
    }
    m->free_hint = m->max_pages;
    return -1;
}

static long alloc_page(VspecRocmPagedMeta* m, int owner) {
    long p = take_first_free(m, owner);
    if (p >= 0) return p;
    if (evict_lru(m, owner)) return take_first_free(m, owner);
    return -1;
}

VspecRocmPagedMeta* vspec_rocm_paged_meta_create(size_t page_tokens, size_t max_pages,
                                                 size_t max_sessions,
                                                 size_t max_pages_per_session) {
    if (page_tokens == 0u || max_pages == 0u || max_pages > UINT32_MAX) return NULL;
    if (max_sessions == 0u) max_sessions = 128u;
    if (max_pages_per_session == 0u) max_pages_per_session = 1024u;
    VspecRocmPagedMeta* m = (VspecRocmPagedMeta*)calloc(1, sizeof(*m));
    if (!m) return NULL;
    m->page_tokens = page_tokens;
    m->max_pages = max_pages;
    m->max_sessions = max_sessions;
    m->max_pages_per_session = max_pages_per_session;
    m->page = (Page*)calloc(max_pages, sizeof(Page));
    m->session = (Session*)calloc(max_sessions, sizeof(Session));
    m->page_lists = (uint32_t*)calloc(max_sessions * max_pages_per_session, sizeof(uint32_t));
    if (!m->page || !m->session || !m->page_lists) {
        vspec_rocm_paged_meta_destroy(m);
        return NULL;
    }
    vspec_rocm_paged_meta_reset(m);
    return m;
}

void vspec_rocm_paged_meta_destroy(VspecRocmPagedMeta* m) {
    if (!m) return;
    free(m->page);
    free(m->session);
    free(m->page_lists);
    free(m->rows);
    free(m->scratch_ids);
    free(m->scratch_slot);
    free(m->scratch_gen);
    free(m);
}

void vspec_rocm_paged_meta_reset(VspecRocmPagedMeta* m) {
    if (!m) return;
    memset(m->page, 0, m->max_pages * sizeof(Page));
    memset(&m->stats, 0, sizeof(m->stats));
    for (size_t i = 0; i < m->max_sessions; ++i) {
        memset(&m->session[i], 0, sizeof(Session));
        m->session[i].pages = m->page_lists + i * m->max_pages_per_session;
    }
    m->clock_step = 1u;
    m->free_hint = 0u;
    /* sessions restart: nothing the planner wrote before can be extended */
    m->rows_tables = NULL;
    m->rows_used = NULL;
    m->rows_max_blocks = 0u;
}

int vspec_rocm_paged_open_session(VspecRocmPagedMeta* m, uint64_t id) {
    if (!m || id == 0u) return 0;
    if (find_session(m, id) >= 0) return 1;
    int slot = find_free_session(m);
    if (slot < 0) {
        if (!evict_lru(m, -1)) return 0;
        slot = find_free_session(m);
        if (slot < 0) return 0;
    }
    m->session[slot].active = 1u;
    m->session[slot].session_id = id;
    m->session[slot].last_touch_step = m->clock_step;
    m->session[slot].gen = ++m->gen_clock;
    return 1;
}

/* the slot of session id, opened if needed (-1: no slot) */
static int open_slot(VspecRocmPagedMeta* m, uint64_t id) {
    int slot = find_session(m, id);
    if (slot >= 0) return slot;
    if (!vspec_rocm_paged_open_session(m, id)) return -1;
    return find_session(m, id);
}

int vspec_rocm_paged_close_session(VspecRocmPagedMeta* m, uint64_t id) {
    const int slot = find_session(m, id);
    if (slot < 0) return 0;
    release_session(m, slot);
    return 1;
}

int vspec_rocm_paged_reuse_prefix(VspecRocmPagedMeta* m, uint64_t target, uint64_t source,
                                  size_t max_tokens) {
    if (!m || target == 0u || source == 0u) return 0;
    const int src = find_session(m, source);
    if (src < 0) return 0;
    if (!vspec_rocm_paged_open_session(m, target)) return 0;
    const int dst = find_session(m, target);
    if (dst < 0) return 0;
    Session* t = &m->session[dst];
    const Session* s = &m->session[src];
    if (t->page_count != 0u) return 0;
    size_t copied = 0;
    for (size_t i = 0; i < s->page_count; ++i) {
        if (t->page_count >= m->max_pages_per_session) break;
        const uint32_t p = s->pages[i];
        if (p >= m->max_pages) continue;
        const size_t used = m->page[p].used_tokens;
        if (max_tokens > 0u && copied >= max_tokens) break;
        if (max_tokens > 0u && copied + used > max_tokens) break;
        t->pages[t->page_count++] = p;
        t->total_tokens += used;
        m->page[p].ref_count += 1u;
        copied += used;
        m->stats.page_reuse_count += 1u;
    }
    t->last_touch_step = m->clock_step;
    return 1;
}

/* The bookkeeping of one append; also reports the page's index in the session's list,
 * which locates the token in table-slot space (index * page_tokens + slot). */
static int reserve_in(VspecRocmPagedMeta* m, int slot, uint32_t* page_out, uint32_t* slot_out,
                      size_t* index_out) {
    Session* s = &m->session[slot];
    m->clock_step += 1u;
    s->last_touch_step = m->clock_step;

    long p = -1;
    if (s->page_count > 0u) {
        p = (long)s->pages[s->page_count - 1u];
        if ((size_t)p >= m->max_pages) p = -1;
    }
    if (p >= 0 && (m->page[p].used_tokens >= m->page_tokens || m->page[p].ref_count > 1u)) p = -1;
    if (p < 0) {
        if (s->page_count >= m->max_pages_per_session) return 0;
        p = alloc_page(m, slot);
        if (p < 0) return 0;
        s->pages[s->page_count++] = (uint32_t)p;
    }
    if (page_out) *page_out = (uint32_t)p;
    if (slot_out) *slot_out = m->page[p].used_tokens;
    if (index_out) *index_out = s->page_count - 1u;
    m->page[p].used_tokens += 1u;
    m->page[p].last_touch_step = m->clock_step;
    s->total_tokens += 1u;
    m->stats.append_token_count += 1u;
    return 1;
}

static int reserve_token(VspecRocmPagedMeta* m, uint64_t id, uint32_t* page_out, uint32_t* slot_out,
                         size_t* index_out) {
    if (!m) return 0;
    const int slot = open_slot(m, id);
    if (slot < 0) return 0;
    return reserve_in(m, slot, page_out, slot_out, index_out);
}

int vspec_rocm_paged_reserve(VspecRocmPagedMeta* m, uint64_t id, uint32_t* page_out, uint32_t* slot_out) {
    return reserve_token(m, id, page_out, slot_out, NULL);
}

int vspec_rocm_paged_locate(const VspecRocmPagedMeta* m, uint64_t id, size_t token_idx,
                            uint32_t* page_out, uint32_t* slot_out) {
    if (!m || !page_out || !slot_out) return 0;
    const int slot = find_session(m, id);
    if (slot < 0) return 0;
    const Session* s = &m->session[slot];
    if (token_idx >= s->total_tokens) return 0;
    size_t remain = token_idx;
    uint32_t page = 0u;  /* a walk that runs off the end lands on page 0, slot 0 (:333-334) */
    size_t in_page = 0u;
    for (size_t i = 0; i < s->page_count; ++i) {
        const uint32_t p = s->pages[i];
        if (p >= m->max_pages) return 0;
        const size_t used = m->page[p].used_tokens;
        if (remain < used) {
            page = p;
            in_page = remain;
            break;
        }
        remain -= used;
    }
    *page_out = page;
    *slot_out = (uint32_t)in_page;
    return 1;
}

size_t vspec_rocm_paged_session_tokens(const VspecRocmPagedMeta* m, uint64_t id) {
    const int slot = find_session(m, id);
    return slot < 0 ? 0u : m->session[slot].total_tokens;
}

void vspec_rocm_paged_stats(const VspecRocmPagedMeta* m, VspecRocmPagedStats* out) {
    if (!m || !out) return;
    *out = m->stats;
    out->free_pages = 0u;
    out->active_sessions = 0u;
    for (size_t i = 0; i < m->max_pages; ++i) {
        if (!m->page[i].allocated) out->free_pages += 1u;
    }
    for (size_t i = 0; i < m->max_sessions; ++i) {
        if (m->session[i].active) out->active_sessions += 1u;
    }
}

size_t vspec_rocm_paged_session_pages(const VspecRocmPagedMeta* m, uint64_t id, uint32_t* out,
                                      size_t cap) {
    const int slot = find_session(m, id);
    if (slot < 0) return 0u;
    const Session* s = &m->session[slot];
    for (size_t i = 0; out && i < s->page_count && i < cap; ++i) out[i] = s->pages[i];
    return s->page_count;
}

int vspec_rocm_paged_page_info(const VspecRocmPagedMeta* m, size_t page, uint32_t* allocated,
                               uint32_t* used_tokens, uint32_t* ref_count) {
    if (!m || page >= m->max_pages) return 0;
    if (allocated) *allocated = m->page[page].allocated;
    if (used_tokens) *used_tokens = m->page[page].used_tokens;
    if (ref_count) *ref_count = m->page[page].ref_count;
    return 1;
}

int vspec_rocm_paged_block_layout(const VspecRocmPagedMeta* m, uint64_t id, int32_t* blocks, int32_t* used,
                                  size_t cap, uint32_t* span, uint32_t* tokens) {
    const int slot = find_session(m, id);
    if (slot < 0 || !blocks || !used) return 0;
    const Session* s = &m->session[slot];
    if (s->page_count > cap) return 0;
    if (s->page_count && s->page_count * m->page_tokens > (size_t)INT32_MAX) return 0;
    uint32_t last_used = 0u;
    for (size_t i = 0; i < s->page_count; ++i) {
        const uint32_t p = s->pages[i];
        if (p >= m->max_pages || p > (uint32_t)INT32_MAX) return 0;
        blocks[i] = (int32_t)p;
        used[i] = (int32_t)m->page[p].used_tokens;
        last_used = m->page[p].used_tokens;
    }
    if (span) *span = s->page_count ? (uint32_t)((s->page_count - 1u) * m->page_tokens + last_used) : 0u;
    if (tokens) *tokens = (uint32_t)s->total_tokens;
    return 1;
}

int vspec_rocm_paged_block_table(const VspecRocmPagedMeta* m, uint64_t id, int32_t* out,
                                 size_t cap, uint32_t* ctx_len) {
    const int slot = find_session(m, id);
    if (slot < 0 || !out) return 0;
    const Session* s = &m->session[slot];
    if (s->page_count > cap || s->total_tokens > (size_t)INT32_MAX) return 0;
    for (size_t i = 0; i < s->page_count; ++i) {
        const uint32_t p = s->pages[i];
        if (p >= m->max_pages || p > (uint32_t)INT32_MAX) return 0;
        if (i + 1u < s->page_count && m->page[p].used_tokens != m->page_tokens) return 0;
        out[i] = (int32_t)p;
    }
    if (ctx_len) *ctx_len = (uint32_t)s->total_tokens;
    return 1;
}

/* Row i of the step tables for session s: entries [from, page_count) written (page ids, and
 * used counts when urow is set), entries [page_count, clear_to) reset to -1 / 0; *ctx the
 * session's token count (plain tables) or its span (with used counts).  Checks everything
 * before it writes, so a refused row is left as it was.  Plain tables need every page but
 * the last to be full; the entries before `from` were checked when they were written. */
static int write_row(const VspecRocmPagedMeta* m, const Session* s, int32_t* row, int32_t* urow,
                     size_t max_blocks, size_t from, size_t clear_to, int32_t* ctx) {
    const size_t n = s->page_count;
    if (n > max_blocks || (n && n * m->page_tokens > (size_t)INT32_MAX) || s->total_tokens > (size_t)INT32_MAX) {
        return 0;
    }
    for (size_t k = from; k < n; ++k) {
        const uint32_t p = s->pages[k];
        if (p >= m->max_pages || p > (uint32_t)INT32_MAX) return 0;
        if (!urow && k + 1u < n && m->page[p].used_tokens != m->page_tokens) return 0;
    }
    for (size_t k = from; k < n; ++k) {
        row[k] = (int32_t)s->pages[k];
        if (urow) urow[k] = (int32_t)m->page[s->pages[k]].used_tokens;
    }
    for (size_t k = n; k < clear_to && k < max_blocks; ++k) {
        row[k] = -1;
        if (urow) urow[k] = 0;
    }
    const size_t last = n ? m->page[s->pages[n - 1u]].used_tokens : 0u;
    *ctx = urow ? (int32_t)(n ? (n - 1u) * m->page_tokens + last : 0u) : (int32_t)s->total_tokens;
    return 1;
}

static int grow_scratch(VspecRocmPagedMeta* m, size_t n) {
    if (n <= m->scratch_cap) return 1;
    const size_t cap = n < 64u ? 64u : n + n / 2u;
    uint64_t* ids = (uint64_t*)realloc(m->scratch_ids, cap * sizeof(uint64_t));
    if (ids) m->scratch_ids = ids;
    int* sl = (int*)realloc(m->scratch_slot, cap * sizeof(int));
    if (sl) m->scratch_slot = sl;
    uint64_t* gn = (uint64_t*)realloc(m->scratch_gen, cap * sizeof(uint64_t));
    if (gn) m->scratch_gen = gn;
    if (!ids || !sl || !gn) return 0;
    m->scratch_cap = cap;
    return 1;
}

static int cmp_u64(const void* a, const void* b) {
    const uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

/* The planner behind vspec_rocm_paged_plan_step (keep = 0: every row written whole) and
 * vspec_rocm_paged_plan_step_update (keep = 1: rows the previous call wrote into the same
 * tables for the same session activation only get their changed entries). */
static int plan(VspecRocmPagedMeta* m, const VspecRocmStepItem* items, size_t n_items, int32_t* block_tables,
                int32_t* block_used, size_t max_blocks, int32_t* ctx_lens, int32_t* start_pos, int32_t* token_item,
                int32_t* token_pos, size_t max_tokens, size_t* n_tokens, int keep) {
    if (!m || (n_items && (!items || !block_tables || !ctx_lens || !start_pos)) || max_blocks == 0) {
        return 0;
    }
    if (!grow_scratch(m, n_items ? n_items : 1u)) return 0;
    size_t total = 0;
    for (size_t i = 0; i < n_items; ++i) {
        if (items[i].token_quota > (size_t)INT32_MAX || total + items[i].token_quota > max_tokens) return 0;
        total += items[i].token_quota;
        m->scratch_ids[i] = items[i].request_id;
    }
    if (total && (!token_item || !token_pos)) return 0;
    /* a repeated request refuses the step before anything is reserved */
    qsort(m->scratch_ids, n_items, sizeof(uint64_t), cmp_u64);
    for (size_t i = 1; i < n_items; ++i) {
        if (m->scratch_ids[i] == m->scratch_ids[i - 1u]) return 0;
    }
    int ok = 1;
    size_t off = 0;
    for (size_t i = 0; ok && i < n_items; ++i) {
        const int slot = open_slot(m, items[i].request_id);
        if (slot < 0) {
            ok = 0;
            break;
        }
        m->scratch_slot[i] = slot;
        m->scratch_gen[i] = m->session[slot].gen;
        for (size_t t = 0; t < items[i].token_quota; ++t) {
            uint32_t in_page = 0u;
            size_t index = 0u;
            if (!reserve_in(m, slot, NULL, &in_page, &index)) {
                ok = 0;
                break;
            }
            const size_t pos = index * m->page_tokens + in_page;
            if (pos > (size_t)INT32_MAX) {
                ok = 0;
                break;
            }
            if (t == 0) start_pos[i] = (int32_t)pos;
            token_item[off + t] = (int32_t)i;
            token_pos[off + t] = (int32_t)pos;
        }
        if (ok && items[i].token_quota == 0u) {
            /* no new token: the next free position in table-slot space */
            const Session* s = &m->session[slot];
            const size_t last = s->page_count ? m->page[s->pages[s->page_count - 1u]].used_tokens : 0u;
            start_pos[i] = (int32_t)(s->page_count ? (s->page_count - 1u) * m->page_tokens + last : 0u);
        }
        off += items[i].token_quota;
    }
    /* what the caller's rows hold: known only for the tables the previous update call wrote */
    const int known = keep && block_tables == m->rows_tables && block_used == m->rows_used &&
                      max_blocks == m->rows_max_blocks;
    if (keep && !known) {
        /* other tables: no row's content is known until this call has written it */
        m->rows_tables = NULL;
        m->rows_used = NULL;
        m->rows_max_blocks = 0u;
        for (size_t i = 0; i < m->rows_cap; ++i) m->rows[i].len = (uint32_t)-1;
    }
    if (keep && n_items > m->rows_cap) {
        const size_t cap = n_items + n_items / 2u;
        RowState* r = (RowState*)realloc(m->rows, cap * sizeof(RowState));
        if (!r) return 0;
        for (size_t i = m->rows_cap; i < cap; ++i) r[i].len = (uint32_t)-1;  /* unknown content */
        m->rows = r;
        m->rows_cap = cap;
    }
    for (size_t i = 0; ok && i < n_items; ++i) {
        const int slot = m->scratch_slot[i];
        const Session* s = &m->session[slot];
        /* an eviction triggered by a later item ended this session's activation */
        if (!s->active || s->gen != m->scratch_gen[i]) {
            ok = 0;
            break;
        }
        int32_t* row = block_tables + i * max_blocks;
        int32_t* urow = block_used ? block_used + i * max_blocks : NULL;
        size_t from = 0u, clear_to = max_blocks;
        if (known && m->rows[i].len != (uint32_t)-1) {
            const RowState* r = &m->rows[i];
            if (r->slot == (uint32_t)slot && r->gen == s->gen && r->len <= s->page_count) {
                from = r->len ? r->len - 1u : 0u;  /* the old last entry's used count may have grown */
                clear_to = 0u;
            } else {
                clear_to = r->len;
            }
        }
        if (!write_row(m, s, row, urow, max_blocks, from, clear_to, &ctx_lens[i])) {
            ok = 0;
            break;
        }
        if (keep) {
            m->rows[i].slot = (uint32_t)slot;
            m->rows[i].gen = s->gen;
            m->rows[i].len = (uint32_t)s->page_count;
        }
    }
    if (keep) {
        if (ok) {
            m->rows_tables = block_tables;
            m->rows_used = block_used;
            m->rows_max_blocks = max_blocks;
        }
    }
    if (ok && n_tokens) *n_tokens = total;
    return ok;
}

/* One continuous-batching step (the items of vspec_continuous_batch_next_batch,
 * continuous_batch.c:155-270): reserve every item's token_quota new tokens, then emit
 * the kernels' inputs.  Items are processed in order; item i's new tokens are packed
 * at [sum of earlier quotas, + quota).  Positions are in table-slot space (page index in
 * the session * page_tokens + slot), which equals the token index while every page but
 * the last is full.  With block_used, every session is expressed (ctx_lens = span,
 * block_used = per-entry used counts); without it, a session whose shared, partly filled
 * page sits in the middle fails the step.  Also fails when an item repeats a request, a
 * reservation fails, a later reservation evicted an earlier item's session, or an output
 * is too small.  Reservations made before a failure stay made, as with a sequence of
 * reference appends that stops at its first failure. */
int vspec_rocm_paged_plan_step(VspecRocmPagedMeta* m, const VspecRocmStepItem* items,
                               size_t n_items, int32_t* block_tables, int32_t* block_used,
                               size_t max_blocks, int32_t* ctx_lens, int32_t* start_pos,
                               int32_t* token_item, int32_t* token_pos, size_t max_tokens,
                               size_t* n_tokens) {
    return plan(m, items, n_items, block_tables, block_used, max_blocks, ctx_lens, start_pos, token_item, token_pos,
                max_tokens, n_tokens, 0);
}

/* The same step over tables the caller keeps between steps: rows that the previous call
 * wrote into the same buffers for the same session (and activation) only get the entries
 * that changed; the others are written whole. */
int vspec_rocm_paged_plan_step_update(VspecRocmPagedMeta* m, const VspecRocmStepItem* items,
                                      size_t n_items, int32_t* block_tables, int32_t* block_used,
                                      size_t max_blocks, int32_t* ctx_lens, int32_t* start_pos,
                                      int32_t* token_item, int32_t* token_pos, size_t max_tokens,
                                      size_t* n_tokens) {
    return plan(m, items, n_items, block_tables, block_used, max_blocks, ctx_lens, start_pos, token_item, token_pos,
                max_tokens, n_tokens, 1);
}
