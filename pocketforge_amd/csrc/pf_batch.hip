// Multi-sequence engine: n independent sequences over one model, decoded
// in lockstep so that every forward pass covers all of them (a verify pass
// of n sequences is n * (n_mtp + 1) rows, which the int8 MFMA GEMM takes in
// one launch per matrix).  Each sequence owns its KV planes, decode state
// (st[s]), token buffer (tokens + s * tok_cap), sampling seed and draw
// counter, so every sequence's tokens equal those of a single-sequence
// engine given the same prompt and seed: every kernel computes each row
// without reference to the rows beside it.
//
// Included at the end of pf_runtime.hip (it uses the engine internals).

// Positions of sequence 0 live in e->pos for the single-sequence API.
static void batch_sync_in(pf_engine* e) { e->spos[0] = e->pos; }
static void batch_sync_out(pf_engine* e) { e->pos = e->spos[0]; }

extern "C" pf_status pf_batch_create(pf_model* m, const pf_cache_desc* cd, uint32_t n_seq, pf_engine** out) {
    return engine_create(m, cd, n_seq, out);
}

extern "C" uint32_t pf_batch_sequences(const pf_engine* e) { return e ? e->nseq : 0; }

extern "C" uint32_t pf_batch_position(const pf_engine* e, uint32_t seq) {
    if (!e || seq >= e->nseq) return 0;
    return seq == 0 ? e->pos : e->spos[seq];
}

// Prompt passes of one sequence: consecutive positions in passes of up to
// one window (at most 256 rows), exactly as pf_generate's prefill.
static pf_status batch_prefill_seq(pf_engine* e, uint32_t seq, const int32_t* tokens, uint32_t n) {
    pf_ctx* c = e->c;
    hipStream_t st = c->stream;
    for (uint32_t i = 0; i < n; i += e->prefill_rows) {
        const uint32_t k = std::min(e->prefill_rows, n - i);
        e->pd_host.pos0 = e->spos[seq];
        e->pd_host.m = k;
        e->pd_host.batch = 0;
        e->pd_host.seq0 = seq;
        for (uint32_t r = 0; r < k; r++) e->pd_host.tok[r] = tokens[i + r];
        PF_HIP(c, hipMemcpyAsync(e->pdP, &e->pd_host, sizeof(PassDesc), hipMemcpyHostToDevice, st));
        // the copy reads e->pd_host before the host overwrites it for the next pass
        PF_HIP(c, hipStreamSynchronize(st));
        if (pf_status s = run_pass(e, e->pdP, k, e->spos[seq], nullptr, nullptr)) return s;
        e->spos[seq] += k;
    }
    e->pd_host.seq0 = 0;
    return PF_OK;
}

static pf_status check_tokens(pf_engine* e, const int32_t* t, size_t n) {
    const uint32_t V = e->m->d.n_vocab;
    for (size_t i = 0; i < n; i++)
        if (t[i] < 0 || (uint32_t)t[i] >= V) return fail(e->c, PF_ERR_ARG, "token id out of range");
    return PF_OK;
}

extern "C" pf_status pf_batch_prefill(pf_engine* e, uint32_t seq, const int32_t* tokens, uint32_t n) {
    if (!e || (!tokens && n) || seq >= e->nseq) return PF_ERR_ARG;
    if (pf_status s = check_tokens(e, tokens, n)) return s;
    batch_sync_in(e);
    if ((uint64_t)e->spos[seq] + n > e->rope_pos)
        return fail(e->c, PF_ERR_CAPACITY, "position beyond the engine's max_context");
    pf_status s = batch_prefill_seq(e, seq, tokens, n);
    batch_sync_out(e);
    if (s) return s;
    PF_HIP(e->c, hipStreamSynchronize(e->c->stream));
    return ll_check(e);
}

extern "C" pf_status pf_batch_forward(pf_engine* e, const uint32_t* seqs, uint32_t n, uint32_t rows_per_seq,
                                      const int32_t* tokens, float* logits, float* hidden) {
    if (!e || !seqs || !tokens || n == 0 || rows_per_seq == 0) return PF_ERR_ARG;
    pf_ctx* c = e->c;
    const pf_model_desc& d = e->m->d;
    const uint32_t rows = n * rows_per_seq;
    const uint32_t out_rows = std::max(MAX_PASS_ROWS, (d.n_mtp + 1) * e->nseq);
    if (rows > e->rows || ((logits || hidden) && rows > out_rows))
        return fail(c, PF_ERR_ARG, "batched pass taller than the engine's pass buffers");
    if (pf_status s = check_tokens(e, tokens, rows)) return s;
    std::vector<uint8_t> seen(e->nseq, 0);
    for (uint32_t i = 0; i < n; i++) {
        if (seqs[i] >= e->nseq || seen[seqs[i]]) return fail(c, PF_ERR_ARG, "sequence ids must be distinct and < n_seq");
        seen[seqs[i]] = 1;
    }
    batch_sync_in(e);
    uint32_t pos_last = 0;
    PassDesc& pd = e->pd_host;
    pd.pos0 = 0;
    pd.m = rows;
    pd.batch = 1;
    pd.seq0 = 0;
    for (uint32_t i = 0; i < n; i++)
        for (uint32_t j = 0; j < rows_per_seq; j++) {
            const uint32_t r = i * rows_per_seq + j;
            pd.tok[r] = tokens[r];
            pd.rpos[r] = e->spos[seqs[i]] + j;
            pd.rseq[r] = seqs[i];
            pos_last = std::max(pos_last, pd.rpos[r]);
        }
    if ((uint64_t)pos_last + 1 > e->rope_pos) return fail(c, PF_ERR_CAPACITY, "position beyond the engine's max_context");
    PF_HIP(c, hipMemcpyAsync(e->pdP, &pd, sizeof(PassDesc), hipMemcpyHostToDevice, c->stream));
    PF_HIP(c, hipStreamSynchronize(c->stream));
    pd.batch = 0;
    e->batch_group = rows_per_seq;           // each sequence's rows_per_seq consecutive positions
    pf_status s = run_pass(e, e->pdP, rows, 0, logits ? e->logitsB : nullptr, hidden ? e->hiddenB : nullptr, true,
                           pos_last);
    e->batch_group = 0;
    if (s) return s;
    for (uint32_t i = 0; i < n; i++) e->spos[seqs[i]] += rows_per_seq;
    batch_sync_out(e);
    if (logits)
        PF_HIP(c, hipMemcpyAsync(logits, e->logitsB, (size_t)rows * d.n_vocab * 4, hipMemcpyDeviceToHost, c->stream));
    if (hidden)
        PF_HIP(c, hipMemcpyAsync(hidden, e->hiddenB, (size_t)rows * d.n_embd * 4, hipMemcpyDeviceToHost, c->stream));
    PF_HIP(c, hipStreamSynchronize(c->stream));
    return ll_check(e);
}

// MTPHeads::forward chain (src/mtp.cpp:63-127) for rows 0..n-1 of h0 (the
// MTP sequences of a batched round), each head's drafts sampled right
// after its logits.
static pf_status batch_mtp_chain(pf_engine* e, const float* h0, uint32_t n, const SamplingCfg& cfg) {
    pf_ctx* c = e->c;
    const pf_model* m = e->m;
    const pf_model_desc& d = m->d;
    hipStream_t st = c->stream;
    const uint32_t D = d.n_embd, V = d.n_vocab, R = d.n_mtp + 1;
    for (uint32_t k = 0; k < d.n_mtp; k++) {
        const float* hin = k == 0 ? h0 : e->mcur;   // head 0 reads the rows of h0 (stride d) itself
        launch_gemv_f32_glu(st, m->mtp[k * 3 + 0], m->mtp[k * 3 + 1], n, hin, D, e->ma, D);
        launch_gemv_f32(st, m->mtp[k * 3 + 2], n, e->ma, D, e->mcur, D, hin);
        launch_gemv_f32(st, m->emb, n, e->mcur, D, e->mlogb, V, nullptr);
        hipLaunchKernelGGL(k_bsample, dim3(n), dim3(1024), 0, st, (const float*)e->mlogb, V, V, cfg,
                           (const uint64_t*)e->seeds, e->st, (const uint32_t*)e->sel, 0u, e->tokens, e->tok_cap,
                           e->pdB, R, (int32_t)ROLE_DRAFT, (int32_t)k);
    }
    PF_LAUNCHED(c);
    return PF_OK;
}

// Engine::generate (src/engine.cpp:276-396) for every sequence at once.
// Prompts are forwarded in order: all but the last 8 tokens of each in
// single-sequence passes, the rest in passes that batch the prompt tails of
// many sequences (a one-token prompt per sequence is one pass); then each
// round runs one
// batched base pass over the unfinished sequences, T1 and the drafts of the
// sequences that take an MTP round (n_gen + 4 <= max_new), one batched
// verify pass over their [T1, drafts] rows, acceptance and correctives, and
// the single-token step of the others.  The host reads the decode states
// back once per round.
// One decode round of the sequences in `cand` that still generate
// (n_gen < lim and not stopped by the memory guard): the MTP sequences
// (src/engine.cpp:304-305: heads on, a stored position, 4 tokens of budget
// left) take the base pass, T1 and drafts, one verify pass of n_mtp + 1 rows
// each, acceptance and the corrective; the others a single-token step; all
// in the same passes.  hs receives every sequence's device state; n_gen,
// have_row, oom and res[q] are updated for the sequences that ran, and
// *ran tells whether any did.
static pf_status batch_round(pf_engine* e, const SamplingCfg& cfg, const std::vector<uint32_t>& cand,
                             const std::vector<uint32_t>& lim, std::vector<uint32_t>& n_gen,
                             std::vector<uint8_t>& have_row, std::vector<uint8_t>& oom, pf_gen_result* res,
                             std::vector<DecodeState>& hs, bool* ran) {
    pf_ctx* c = e->c;
    const pf_model_desc& d = e->m->d;
    hipStream_t st = c->stream;
    const uint32_t N = e->nseq, V = d.n_vocab, NM = d.n_mtp, R = NM + 1;
    std::vector<uint32_t> sel(N);
    *ran = false;
    // MTP sequences first (src/engine.cpp:304-305), then single-token steps
    uint32_t nm = 0, na = 0, pos_hi = 0;
    const bool out_of_memory = e->max_memory && c->bytes > e->max_memory;   // src/engine.cpp:297-301
    for (int pass = 0; pass < 2; pass++)
        for (const uint32_t s : cand) {
            if (n_gen[s] >= lim[s] || oom[s]) continue;
            if (out_of_memory) { oom[s] = 1; continue; }
            const bool mtp = e->mtp_enabled && NM > 0 && e->spos[s] > 0 && n_gen[s] + 4 <= lim[s];
            if (mtp != (pass == 0)) continue;
            sel[na++] = s;
            if (mtp) nm++;
            pos_hi = std::max(pos_hi, e->spos[s]);
        }
    if (na == 0) return PF_OK;
    *ran = true;
    if ((uint64_t)pos_hi + NM + 2 > e->rope_pos) return fail(c, PF_ERR_CAPACITY, "position beyond the engine's max_context");
    e->timed_used = 0;
    e->kev_used = 0;
    PF_HIP(c, hipMemcpyAsync(e->sel, sel.data(), (size_t)na * 4, hipMemcpyHostToDevice, st));
    PF_HIP(c, hipEventRecord(e->rev0, st));
    hipLaunchKernelGGL(k_bctl_pass_a, dim3(1), dim3(256), 0, st, e->st, (const uint32_t*)e->sel, na, e->pdA);
    TimedPass* tp = nullptr;
    pf_status s;
    if ((s = timed_begin(e, false, &tp))) return s;
    if ((s = run_pass(e, e->pdA, na, 0, e->logitsA, e->hiddenA, true, pos_hi))) return s;
    if (tp) PF_HIP(c, hipEventRecord(tp->b, st));
    if (nm) {
        hipLaunchKernelGGL(k_bsample, dim3(nm), dim3(1024), 0, st, (const float*)e->logitsA, V, V, cfg,
                           (const uint64_t*)e->seeds, e->st, (const uint32_t*)e->sel, 0u, e->tokens, e->tok_cap,
                           e->pdB, R, (int32_t)ROLE_T1, 0);
        if ((s = batch_mtp_chain(e, e->hiddenA, nm, cfg))) return s;
        if ((s = timed_begin(e, true, &tp))) return s;
        e->in_verify = true;
        e->batch_group = R;                      // each MTP sequence's R verify rows
        s = run_pass(e, e->pdB, nm * R, 0, e->logitsB, nullptr, true, pos_hi + R);
        e->batch_group = 0;
        e->in_verify = false;
        if (s) return s;
        if (tp) PF_HIP(c, hipEventRecord(tp->b, st));
        hipLaunchKernelGGL(k_bargmax_rows, dim3(nm * R), dim3(1024), 0, st, (const float*)e->logitsB, V, R,
                           (const uint32_t*)e->sel, e->st);
        hipLaunchKernelGGL(k_bctl_accept, dim3((nm + 63) / 64), dim3(64), 0, st, e->st, (const uint32_t*)e->sel,
                           nm, (const PassDesc*)e->pdB, R, e->tokens, e->tok_cap);
        if (e->skip_on) launch_skip_commit(e, e->pdB, nm * R, 0, 0, true);
        hipLaunchKernelGGL(k_bsample, dim3(nm), dim3(1024), 0, st, (const float*)e->logitsB, V, V, cfg,
                           (const uint64_t*)e->seeds, e->st, (const uint32_t*)e->sel, 0u, e->tokens, e->tok_cap,
                           e->pdB, R, (int32_t)ROLE_CORRECTIVE, 0);
    }
    if (na > nm)
        hipLaunchKernelGGL(k_bsample, dim3(na - nm), dim3(1024), 0, st, (const float*)e->logitsA, V, V, cfg,
                           (const uint64_t*)e->seeds, e->st, (const uint32_t*)e->sel, nm, e->tokens, e->tok_cap,
                           e->pdB, R, (int32_t)ROLE_FALLBACK, 0);
    PF_LAUNCHED(c);
    PF_HIP(c, hipEventRecord(e->rev1, st));
    PF_HIP(c, hipMemcpyAsync(hs.data(), e->st, (size_t)N * sizeof(DecodeState), hipMemcpyDeviceToHost, st));
    PF_HIP(c, hipStreamSynchronize(st));
    if ((s = harvest_events(e, 0, e->timed_used, 0, e->kev_used))) return s;
    if (nm) {
        float ms = 0;
        PF_HIP(c, hipEventElapsedTime(&ms, e->rev0, e->rev1));
        e->round_us += ms * 1000.0;
        e->round_n++;
    }
    for (uint32_t i = 0; i < na; i++) {
        const uint32_t q = sel[i];
        const bool mtp = i < nm;
        res[q].passes += (have_row[q] ? 0 : 1) + (mtp ? 1 : 0);
        if (mtp) {
            res[q].rounds++;
            have_row[q] = (hs[q].round_word & 0xFFu) >= NM;
        } else {
            have_row[q] = 0;
        }
        n_gen[q] = hs[q].n_gen;
        e->spos[q] = hs[q].pos;
    }
    return PF_OK;
}

// ---------------------------------------------------- continuous batching

// A session of sequences that join and leave between rounds; each one's
// tokens equal Engine::generate for its prompt and seed (src/engine.cpp:
// 276-396) whatever else runs beside it.
extern "C" pf_status pf_batch_open(pf_engine* e, const pf_sampling* cfg, uint32_t tokens_cap) {
    if (!e || tokens_cap == 0) return PF_ERR_ARG;
    const uint32_t N = e->nseq;
    if (e->tok_cap != tokens_cap || e->tok_alloc < (size_t)N * tokens_cap)
        if (pf_status s = ensure_tokens(e, tokens_cap)) return s;
    e->bs_cfg = to_cfg(cfg);
    e->bs_state.assign(N, 0);
    e->bs_have.assign(N, 0);
    e->bs_oom.assign(N, 0);
    e->bs_ngen.assign(N, 0);
    e->bs_lim.assign(N, 0);
    e->bs_res.assign(N, pf_gen_result{});
    e->bs_hs.assign(N, DecodeState{});
    e->round_us = 0;
    e->round_n = 0;
    e->bs_open = true;
    return PF_OK;
}

extern "C" pf_status pf_batch_admit(pf_engine* e, uint32_t seq, const int32_t* prompt, uint32_t n_prompt,
                                    uint32_t max_new, uint64_t seed) {
    if (!e || !prompt || n_prompt == 0) return PF_ERR_ARG;
    pf_ctx* c = e->c;
    if (!e->bs_open) return fail(c, PF_ERR_STATE, "pf_batch_open first");
    if (seq >= e->nseq) return fail(c, PF_ERR_ARG, "sequence slot out of range");
    if (e->bs_state[seq] != 0) return fail(c, PF_ERR_STATE, "sequence slot in use (pf_batch_take frees it)");
    if (e->skip_on) return fail(c, PF_ERR_UNSUPPORTED, "continuous batching with layer skip on");
    if (pf_status s = check_tokens(e, prompt, n_prompt)) return s;
    if ((uint64_t)n_prompt + max_new + 1 > e->tok_cap) return fail(c, PF_ERR_CAPACITY, "tokens_cap < prompt + max_new + 1");
    if ((uint64_t)n_prompt + max_new + MAX_PASS_ROWS > e->rope_pos)
        return fail(c, PF_ERR_CAPACITY, "prompt + max_new_tokens exceed the engine's max_context");
    hipStream_t st = c->stream;
    batch_sync_in(e);
    e->spos[seq] = 0;   // a new request starts an empty cache in this slot
    PF_HIP(c, hipMemcpyAsync(e->tokens + (size_t)seq * e->tok_cap, prompt, (size_t)n_prompt * 4,
                             hipMemcpyHostToDevice, st));
    PF_HIP(c, hipMemcpyAsync(e->seeds + seq, &seed, 8, hipMemcpyHostToDevice, st));
    pf_status s = batch_prefill_seq(e, seq, prompt, n_prompt);
    if (s) { batch_sync_out(e); return s; }
    DecodeState h{};
    h.pos = e->spos[seq];
    h.cur = prompt[n_prompt - 1];
    h.n_tokens = n_prompt;
    e->bs_hs[seq] = h;
    PF_HIP(c, hipMemcpyAsync(e->st + seq, &e->bs_hs[seq], sizeof(DecodeState), hipMemcpyHostToDevice, st));
    PF_HIP(c, hipStreamSynchronize(st));
    batch_sync_out(e);
    e->bs_state[seq] = 1;
    e->bs_have[seq] = 0;
    e->bs_oom[seq] = 0;
    e->bs_ngen[seq] = 0;
    e->bs_lim[seq] = max_new;
    e->bs_res[seq] = pf_gen_result{};
    return ll_check(e);
}

extern "C" pf_status pf_batch_step(pf_engine* e, uint32_t* finished, uint32_t* n_finished) {
    if (!e || !n_finished) return PF_ERR_ARG;
    pf_ctx* c = e->c;
    *n_finished = 0;
    if (!e->bs_open) return fail(c, PF_ERR_STATE, "pf_batch_open first");
    std::vector<uint32_t> cand;
    for (uint32_t q = 0; q < e->nseq; q++)
        if (e->bs_state[q] == 1) cand.push_back(q);
    bool ran = false;
    if (!cand.empty()) {
        batch_sync_in(e);
        pf_status s = batch_round(e, e->bs_cfg, cand, e->bs_lim, e->bs_ngen, e->bs_have, e->bs_oom, e->bs_res.data(),
                                  e->bs_hs, &ran);
        batch_sync_out(e);
        if (s) return s;
    }
    for (const uint32_t q : cand) {
        if (e->bs_ngen[q] >= e->bs_lim[q] || e->bs_oom[q]) {
            e->bs_state[q] = 2;
            if (finished) finished[*n_finished] = q;
            (*n_finished)++;
        }
    }
    return ran ? ll_check(e) : PF_OK;
}

extern "C" pf_status pf_batch_take(pf_engine* e, uint32_t seq, int32_t* tokens_out, uint32_t tokens_cap,
                                   pf_gen_result* res) {
    if (!e || !tokens_out || !res) return PF_ERR_ARG;
    pf_ctx* c = e->c;
    if (!e->bs_open) return fail(c, PF_ERR_STATE, "pf_batch_open first");
    if (seq >= e->nseq || e->bs_state[seq] == 0) return fail(c, PF_ERR_STATE, "no sequence in that slot");
    const DecodeState& h = e->bs_hs[seq];
    const uint32_t nt = std::min(std::min(h.n_tokens, e->tok_cap), tokens_cap);
    PF_HIP(c, hipMemcpy(tokens_out, e->tokens + (size_t)seq * e->tok_cap, (size_t)nt * 4, hipMemcpyDeviceToHost));
    *res = e->bs_res[seq];
    res->n_tokens = nt;
    res->mtp_accepted = (int32_t)h.accepted;
    res->mtp_rejected = (int32_t)h.rejected;
    res->oom_protected = e->bs_oom[seq];
    e->bs_state[seq] = 0;
    return PF_OK;
}

extern "C" pf_status pf_batch_generate(pf_engine* e, const int32_t* prompts, const uint32_t* prompt_lens,
                                       uint32_t max_new, const pf_sampling* scfg, const uint64_t* seeds,
                                       int32_t* tokens_out, uint32_t tokens_cap, pf_gen_result* res) {
    if (!e || !prompt_lens || !seeds || !tokens_out || !res) return PF_ERR_ARG;
    pf_ctx* c = e->c;
    const pf_model_desc& d = e->m->d;
    hipStream_t st = c->stream;
    const uint32_t N = e->nseq, V = d.n_vocab, NM = d.n_mtp, R = NM + 1;
    size_t total = 0;
    for (uint32_t s = 0; s < N; s++) total += prompt_lens[s];
    if (total && !prompts) return PF_ERR_ARG;
    if (pf_status s = check_tokens(e, prompts, total)) return s;
    batch_sync_in(e);
    for (uint32_t s = 0; s < N; s++) {
        std::memset(&res[s], 0, sizeof(pf_gen_result));
        if ((uint64_t)prompt_lens[s] + max_new + 1 > tokens_cap)
            return fail(c, PF_ERR_CAPACITY, "tokens_cap < prompt + max_new + 1");
        if ((uint64_t)e->spos[s] + prompt_lens[s] + max_new + MAX_PASS_ROWS > e->rope_pos)
            return fail(c, PF_ERR_CAPACITY, "prompt + max_new_tokens exceed the engine's max_context");
    }
    const SamplingCfg cfg = to_cfg(scfg);
    if (e->tok_cap != tokens_cap || e->tok_alloc < (size_t)N * tokens_cap) {
        if (pf_status s = ensure_tokens(e, tokens_cap)) return s;
    }
    PF_HIP(c, hipMemcpyAsync(e->seeds, seeds, (size_t)N * 8, hipMemcpyHostToDevice, st));
    {
        size_t off = 0;
        for (uint32_t s = 0; s < N; s++) {
            if (prompt_lens[s])
                PF_HIP(c, hipMemcpyAsync(e->tokens + (size_t)s * tokens_cap, prompts + off,
                                         (size_t)prompt_lens[s] * 4, hipMemcpyHostToDevice, st));
            off += prompt_lens[s];
        }
    }
    auto t0 = std::chrono::steady_clock::now();
    std::vector<DecodeState> hs(N);
    {
        // long prompts in single-sequence passes (their rows share one KV
        // list), the last <= 8 tokens of every prompt in batched passes
        std::vector<size_t> off(N + 1, 0);
        for (uint32_t s = 0; s < N; s++) off[s + 1] = off[s] + prompt_lens[s];
        std::vector<uint32_t> tail(N);
        for (uint32_t s = 0; s < N; s++) {
            const uint32_t head = prompt_lens[s] > MAX_PASS_ROWS ? prompt_lens[s] - MAX_PASS_ROWS : 0;
            tail[s] = prompt_lens[s] - head;
            if (pf_status r = batch_prefill_seq(e, s, prompts + off[s], head)) { batch_sync_out(e); return r; }
        }
        PassDesc& pd = e->pd_host;
        for (uint32_t s0 = 0; s0 < N;) {
            uint32_t rows = 0, pos_last = 0, s1 = s0;
            for (; s1 < N && rows + tail[s1] <= e->rows; s1++) {
                const uint32_t head = prompt_lens[s1] - tail[s1];
                for (uint32_t j = 0; j < tail[s1]; j++, rows++) {
                    pd.tok[rows] = prompts[off[s1] + head + j];
                    pd.rpos[rows] = e->spos[s1] + j;
                    pd.rseq[rows] = s1;
                    pos_last = std::max(pos_last, pd.rpos[rows]);
                }
            }
            if (rows) {
                pd.pos0 = 0;
                pd.m = rows;
                pd.batch = 1;
                pd.seq0 = 0;
                PF_HIP(c, hipMemcpyAsync(e->pdP, &pd, sizeof(PassDesc), hipMemcpyHostToDevice, st));
                PF_HIP(c, hipStreamSynchronize(st));
                pd.batch = 0;
                if (pf_status r = run_pass(e, e->pdP, rows, 0, nullptr, nullptr, true, pos_last)) {
                    batch_sync_out(e);
                    return r;
                }
                for (uint32_t s = s0; s < s1; s++) e->spos[s] += tail[s];
            }
            s0 = s1;
        }
        for (uint32_t s = 0; s < N; s++) {
            hs[s] = DecodeState{};
            hs[s].pos = e->spos[s];
            hs[s].cur = prompt_lens[s] ? prompts[off[s] + prompt_lens[s] - 1] : 0;
            hs[s].n_tokens = prompt_lens[s];
        }
    }
    PF_HIP(c, hipMemcpyAsync(e->st, hs.data(), (size_t)N * sizeof(DecodeState), hipMemcpyHostToDevice, st));
    PF_HIP(c, hipStreamSynchronize(st));
    auto t1 = std::chrono::steady_clock::now();

    e->verify_us = e->base_us = 0;
    e->verify_n = e->base_n = 0;
    e->kev_us = e->kev_bytes_sum = 0;
    e->kev_n = 0;
    e->aev_us = 0;
    e->aev_n = 0;
    e->aev_used = 0;
    e->round_us = 0;
    e->round_n = 0;
    std::vector<uint32_t> n_gen(N, 0), lim(N, max_new), cand(N);
    std::vector<uint8_t> have_row(N, 0), oom(N, 0);
    for (uint32_t q = 0; q < N; q++) cand[q] = q;
    for (;;) {
        bool ran = false;
        if (pf_status s = batch_round(e, cfg, cand, lim, n_gen, have_row, oom, res, hs, &ran)) {
            batch_sync_out(e);
            return s;
        }
        if (!ran) break;
    }
    auto t2 = std::chrono::steady_clock::now();
    batch_sync_out(e);
    const double ps = std::chrono::duration<double>(t1 - t0).count();
    const double ds = std::chrono::duration<double>(t2 - t1).count();
    for (uint32_t s = 0; s < N; s++) {
        const uint32_t nt = std::min(hs[s].n_tokens, tokens_cap);
        PF_HIP(c, hipMemcpy(tokens_out + (size_t)s * tokens_cap, e->tokens + (size_t)s * tokens_cap, (size_t)nt * 4,
                            hipMemcpyDeviceToHost));
        res[s].n_tokens = nt;
        res[s].mtp_accepted = (int32_t)hs[s].accepted;
        res[s].mtp_rejected = (int32_t)hs[s].rejected;
        res[s].oom_protected = oom[s];
        res[s].prefill_seconds = ps;
        res[s].decode_seconds = ds;
    }
    return ll_check(e);
}
