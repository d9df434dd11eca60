"""Step packing: SchedulerOutput-shaped plans to device metadata."""
