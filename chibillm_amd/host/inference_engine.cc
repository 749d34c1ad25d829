#include "inference_engine.h"

namespace chibillm {

result<inference_engine, inference_engine_error>
inference_engine::make(scheduler_config config, model_runner& runner)
{
    auto state = runner.make_state(config);
    if (!state)
        return fail(inference_engine_errc::scheduler_creation_failed, state.error(),
                    "create model state");
    auto s = scheduler::make(config, runner.info().eos_token, std::move(*state));
    if (!s)
        return fail(inference_engine_errc::scheduler_creation_failed, s.error());
    return inference_engine(std::move(*s), runner);
}

result<void, inference_engine_error>
inference_engine::add(seq sequence)
{
    auto added = scheduler_.add(std::move(sequence));
    if (!added)
        return fail(inference_engine_errc::sequence_add_failed, added.error());
    return {};
}

result<admission_result, inference_engine_error>
inference_engine::try_add(seq& sequence)
{
    auto admitted = scheduler_.try_add(sequence);
    if (!admitted)
        return fail(inference_engine_errc::sequence_add_failed, admitted.error());
    return *admitted;
}

result<std::vector<sequence_update>, inference_engine_error>
inference_engine::step()
{
    auto scheduled = scheduler_.schedule();
    if (!scheduled)
        return fail(inference_engine_errc::scheduling_failed, scheduled.error());
    auto batch = build_model_batch(*scheduled, scheduler_);
    if (!batch)
        return fail_after_abort(*scheduled, { inference_engine_errc::model_batch_build_failed,
                                              describe_error(batch.error()) });
    auto begun = scheduler_.begin_execution(*batch);
    if (!begun)
        return fail_after_abort(*scheduled, { inference_engine_errc::model_execution_failed,
                                              "begin batch: " + describe_error(begun.error()) });
    auto samples = runner_->execute(*batch, scheduler_.state());
    if (!samples)
        return fail_after_abort(*scheduled, { inference_engine_errc::model_execution_failed,
                                              describe_error(samples.error()) });
    if (samples->size() != batch->sample_count())
        return fail_after_abort(
            *scheduled, { inference_engine_errc::runner_result_count_mismatch,
                          "expected " + std::to_string(batch->sample_count()) + " samples, received "
                              + std::to_string(samples->size()) });
    auto completed = scheduler_.complete(scheduled->id, *samples);
    if (!completed)
        return fail_after_abort(*scheduled, { inference_engine_errc::batch_completion_failed,
                                              describe_error(completed.error()) });
    return std::move(*completed);
}

result<void, inference_engine_error>
inference_engine::cancel(seq_id id)
{
    auto cancelled = scheduler_.cancel(id);
    if (!cancelled)
        return fail(inference_engine_errc::sequence_cancel_failed, cancelled.error());
    return {};
}

result<void, inference_engine_error>
inference_engine::remove(seq_id id)
{
    auto removed = scheduler_.remove(id);
    if (!removed)
        return fail(inference_engine_errc::sequence_remove_failed, removed.error());
    return {};
}

failure<inference_engine_error>
inference_engine::fail_after_abort(const scheduled_batch& batch, inference_engine_error e)
{
    auto aborted = scheduler_.abort(batch.id);
    if (!aborted)
        return fail(inference_engine_error { inference_engine_errc::batch_abort_failed,
                                             describe_error(aborted.error())
                                                 + "; original failure: " + describe_error(e) });
    return fail(std::move(e));
}

} // namespace chibillm
