/* C-ABI access to the reference's BERT embedding and vector memory
 * (fast/vdb.cpp), compiled from the reference's own unmodified source where
 * it lies: this file includes it (oracle/Makefile passes -I to the
 * reference's directory) so that its file-static bert_tokenize (:75-121),
 * bert_embed (:123-245) and the vector memory m_vdb can be reached.  TEST
 * INFRASTRUCTURE ONLY: the checker for the GPU embedding and search, never
 * part of the product path.
 *
 *   ref_bert_open      vdb_set_model + ensure_bert (:52-73)
 *   ref_bert_tokenize  bert_tokenize
 *   ref_bert_embed     bert_embed (mean-pooled, L2-normalised fp32)
 *   ref_vdb_create     vdb_create (:269-335) -> number of entries
 *   ref_vdb_entry      an entry's timestamp and fp16 vector
 *   ref_vdb_query      vdb_query (:337-377) -> indices of the entries found
 */
#include "vdb.cpp"

extern "C" {

int ref_bert_open(const char* fn)
{
    vdb_set_model(fn);
    return ensure_bert() ? 0 : -1;
}

int ref_bert_n_embed(void) { return m_brt.ready ? m_brt.m.n_embed : 0; }

int ref_bert_tokenize(const char* text, int* out, int cap)
{
    const vector<int> t = bert_tokenize(text);
    for (int i = 0; i < (int)t.size() && i < cap; i++) out[i] = t[i];
    return (int)t.size();
}

int ref_bert_embed(const char* text, float* out, int cap)
{
    ftensor e;
    bert_embed(text, e);
    for (int i = 0; i < (int)e.size() && i < cap; i++) out[i] = e[i];
    return (int)e.size();
}

int ref_vdb_create(const char* log)
{
    vdb_create(log);
    return (int)m_vdb.size();
}

int ref_vdb_entry(int i, uint32_t* ts, uint16_t* vec, int cap)
{
    if (i < 0 || i >= (int)m_vdb.size()) return -1;
    const vdb_entry& e = m_vdb[i];
    *ts = e.timestamp;
    for (int j = 0; j < (int)e.vec.size() && j < cap; j++) memcpy(&vec[j], &e.vec[j], 2);
    return (int)e.vec.size();
}

/* the entries vdb_query returns, as indices into m_vdb (matched by their
 * timestamp and text, unique in the logs the tests write) */
int ref_vdb_query(const char* text, int* idx, int cap)
{
    const vecdb r = vdb_query(text);
    int n = 0;
    for (const vdb_entry& e : r) {
        int found = -1;
        for (int i = 0; i < (int)m_vdb.size(); i++)
            if (m_vdb[i].timestamp == e.timestamp && m_vdb[i].user_text == e.user_text &&
                m_vdb[i].context_before == e.context_before && m_vdb[i].context_after == e.context_after) {
                found = i;
                break;
            }
        if (n < cap) idx[n] = found;
        n++;
    }
    return n;
}

} /* extern "C" */
